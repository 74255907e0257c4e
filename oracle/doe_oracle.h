/*
 * doe_oracle.h -- CPU oracle for the quantized-decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference's
 * CPU evaluation of each hot-path kernel (the TSIR reference interpreter, the
 * CSL/WebGPU emulator's CPU backend and the Doppler RDRR Q4_K decoder).  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
 * and only to check results.  The product library (doe_amd) never calls it.
 *
 * Numerics: every function runs single-threaded, in the reference's strict
 * order (f32 left-fold accumulation unless noted), built with
 * -O2 -ffp-contract=off and no fast-math.
 *
 * All functions return 0 on success and a negative value on invalid sizes.
 */
#ifndef DOE_ORACLE_H
#define DOE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions ------------------------------------------------ */
float ora_f16_to_f32(uint16_t h);
uint16_t ora_f32_to_f16(float f);          /* round to nearest even */
float ora_bf16_to_f32(uint16_t h);
uint16_t ora_f32_to_bf16(float f);         /* RNE, NaN kept quiet */

/* ---- Q4_K (144-byte block, 256 weights) ---------------------------------- */
void ora_q4k_unpack_scale_min(const uint8_t *block, uint8_t sc[8], uint8_t mn[8],
                              float *d, float *dmin);
void ora_q4k_dequant_block(const uint8_t *block, float out[256]);
int ora_q4k_dequant_rowwise(const uint8_t *w, int64_t rows, int64_t cols, float *out);
int ora_q4k_gemv(const uint8_t *w, const float *x, float *y, int64_t n, int64_t k);
int ora_q4k_gemv_rows(const uint8_t *w, const float *x, float *y, int64_t n, int64_t k,
                      int64_t row_begin, int64_t row_end);
int ora_q4k_gemm_sampled(const uint16_t *a_bf16, const uint8_t *b, int64_t m, int64_t n,
                         int64_t k, const int64_t *mi, const int64_t *ni, int64_t count,
                         float *out);
int ora_q4k_gemm(const uint16_t *a_bf16, const uint8_t *b, float *c, int64_t m, int64_t n,
                 int64_t k);

/* ---- dense GEMVs --------------------------------------------------------- */
int ora_f32_gemv(const float *w, const float *x, float *y, int64_t m, int64_t k);
int ora_lm_head_gemv(const float *a, const uint16_t *b, float *c, int64_t m, int64_t n,
                     int64_t k, float alpha, int transpose_b);
int ora_f16_gemv(const uint16_t *b, const float *a, float *c, int64_t n, int64_t k,
                 float alpha);
int ora_int4g32_gemv(const uint32_t *q, const uint16_t *scales, const float *x, float *y,
                     int64_t m, int64_t n, int64_t k);
/* Q8_0 (34-byte blocks: f16 scale, 32 int8 quants).  element_count returns
 * the dequantised element count of a buffer, or -1 where the reference's
 * validator rejects its size; dequant and gemv read row-wise Q8_0 rows of
 * ceil(k / 32) blocks. */
int64_t ora_q8_0_element_count(int64_t bytes);
int ora_q8_0_dequant(const uint8_t *w, float *out, int64_t n, int64_t k);
int ora_q8_0_gemv(const uint8_t *w, const float *x, const float *residual, float *y, int64_t n,
                  int64_t k);

/* ---- elementwise / normalisation ---------------------------------------- */
int ora_rmsnorm(const float *x, const float *w, float *out, int64_t rows, int64_t h,
                float eps, int weight_offset);
int ora_rope_table(float *freq_cis, int64_t max_pos, int64_t head_dim, double base);
int ora_rope(float *qk, const float *freq_cis, int64_t seq_len, int64_t num_heads,
             int64_t head_dim, int64_t position_offset);
int ora_rope_pairs(float *x, const float *cos_t, const float *sin_t, int64_t head_dim,
                   int64_t num_pairs, int interleaved);
int ora_geglu(const float *gate, const float *up, float *out, int64_t n);
int ora_residual(const float *a, const float *b, float *out, int64_t n);
int64_t ora_argmax(const float *logits, int64_t n);
int ora_embed_gather(const uint16_t *table_f16, const int32_t *ids, float *out,
                     int64_t n_ids, int64_t vocab, int64_t hidden, float scale);
int ora_gather_f32(const uint32_t *ids, const float *table, float *out, int64_t n_ids,
                   int64_t vocab, int64_t hidden);
int ora_kv_write(const float *k_proj, const float *v_proj, uint16_t *k_cache,
                 uint16_t *v_cache, int64_t num_kv_heads, int64_t max_seq, int64_t head_dim,
                 int64_t pos, int kv_layout);

/* ---- attention ------------------------------------------------------------
 * kv_layout 0: [kv_head][pos][dim]   kv_layout 1: [pos][kv_head][dim]
 * q is [num_heads][head_dim] (decode) or [q_len][num_heads][head_dim] (prefill).
 */
int ora_attn_decode(const float *q, const uint16_t *k, const uint16_t *v, float *o,
                    int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                    int64_t kv_len, int64_t kv_stride, float scale, float softcap,
                    int64_t sliding_window, int kv_layout);
int ora_attn_prefill(const float *q, const float *k, const float *v, float *o,
                     int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                     int64_t q_len, int64_t kv_len, int64_t start_pos, float scale,
                     int causal, int64_t row_begin, int64_t row_end);

/* ---- Qwen 3.6 graph ops (gated DeltaNet body, gated activations) ---------- */
int ora_gated(const float *gate, const float *input, float *out, int64_t n, int kind);
int ora_l2_normalize(const float *in, float *out, int64_t rows, int64_t hidden, float eps);
int ora_conv1d_depthwise(const float *in, const float *w, const float *bias, float *out, int64_t tokens,
                         int64_t channels, int64_t kernel_size);
int ora_linear_attention(const float *q, const float *k, const float *v, const float *gate, float *state,
                         float *out, int64_t tokens, int64_t heads, int64_t key_dim, int64_t value_dim,
                         const float *a_log);

#ifdef __cplusplus
}
#endif

#endif
