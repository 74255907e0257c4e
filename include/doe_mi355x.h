/*
 * doe_mi355x.h -- C ABI of the MI355X (gfx950) quantized-decode hot path.
 *
 * Each compute entry point replaces ONE dispatch of one reference kernel: the
 * reference binds buffers to a WGSL bind group, writes a Uniforms struct and
 * calls wgpuComputePassEncoderDispatchWorkgroups through its webgpu.h drop-in
 * (runtime/zig/src/dropin/dropin_abi_procs.zig:232 SetBindGroup, :237
 * DispatchWorkgroups, :309 QueueSubmit), or memcpy_h2d -> launch("compute") ->
 * memcpy_d2h on the CSL lane (bench/runners/csl-runners/
 * fused_gemv_dequant_sim_runner.py:96-118).  Here each binding becomes a
 * plain device pointer and each Uniforms field a scalar argument, keeping the
 * reference's binding roles, block layouts and shape parameters.
 *
 * Conventions
 *   - Every function returns DOE_OK (0) or a negative DOE_E_* status; the
 *     message of the last failure on the calling thread is doe_last_error().
 *   - Pointers passed to compute entry points are device pointers owned by
 *     the caller (doe_malloc or any hipMalloc'd memory).  The library owns no
 *     per-call state; kernels are re-entrant per stream.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream).  Compute
 *     entry points are asynchronous; errors in arguments are reported
 *     synchronously, device faults at the next synchronising call.
 *   - Sizes are int64_t element counts unless named *_bytes.
 */
#ifndef DOE_MI355X_H
#define DOE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DOE_OK 0
#define DOE_E_INVALID (-1)     /* bad argument (shape, alignment, null) */
#define DOE_E_NOT_INIT (-2)    /* doe_init was not called */
#define DOE_E_HIP (-3)         /* HIP runtime error */
#define DOE_E_UNSUPPORTED (-4) /* valid but unsupported configuration */
#define DOE_E_OOM (-5)         /* device allocation failed */

typedef void *doe_stream_t; /* hipStream_t */
typedef void *doe_event_t;  /* hipEvent_t */
typedef void *doe_graph_t;  /* hipGraphExec_t */

/* ---- lifecycle ------------------------------------------------------------
 * Replaces the drop-in's instance/adapter/device acquisition
 * (runtime/zig/src/dropin/dropin_abi_procs.zig:156-170 region) for one GPU. */
int doe_init(int device);
int doe_shutdown(void);
const char *doe_last_error(void);
/* Writes a JSON object describing the device (name, arch, CUs, clocks). */
int doe_device_info(char *buf, size_t buf_bytes);
int doe_device_synchronize(void);

/* ---- memory ----------------------------------------------------------------
 * Replaces wgpuDeviceCreateBuffer (dropin_abi_procs.zig:156) and
 * wgpuQueueWriteBuffer (:326) / buffer map-read for readback. */
int doe_malloc(void **ptr, size_t bytes);
int doe_free(void *ptr);
int doe_memcpy_h2d(void *dst, const void *src, size_t bytes);
int doe_memcpy_d2h(void *dst, const void *src, size_t bytes);
int doe_memcpy_d2d(void *dst, const void *src, size_t bytes, doe_stream_t stream);
/* `rows` rows of `row_bytes` from src (rows `src_pitch` bytes apart) to dst
 * (rows `dst_pitch` apart), device to device, on `stream`.  No counterpart
 * in the reference: the decoder's batched prompt takes each layer's slice
 * of the per-layer inputs with it. */
int doe_memcpy2d_d2d(void *dst, size_t dst_pitch, const void *src, size_t src_pitch, size_t row_bytes,
                     size_t rows, doe_stream_t stream);
int doe_memset(void *dst, int value, size_t bytes, doe_stream_t stream);

/* ---- streams, events, graphs -----------------------------------------------
 * Replace queue submission (dropin_abi_procs.zig:309) and the timestamp
 * queries of runtime/zig/src/doe_query_native.zig.  Streams are created at
 * the default priority. */
int doe_stream_create(doe_stream_t *stream);
int doe_stream_destroy(doe_stream_t stream);
int doe_stream_synchronize(doe_stream_t stream);
int doe_event_create(doe_event_t *event);
int doe_event_destroy(doe_event_t event);
int doe_event_record(doe_event_t event, doe_stream_t stream);
int doe_event_synchronize(doe_event_t event);
int doe_event_elapsed_ms(float *ms, doe_event_t start, doe_event_t end);
/* Stores the device's constant-rate wall clock (ticks of
 * doe_device_timestamp_hz) to *dst when the stream reaches it: a kernel, so
 * it can sit between the kernels of a captured graph, where event records
 * cannot be timed (doe_event_elapsed_ms rejects events recorded inside a
 * graph).  Measurement utility; no reference counterpart. */
int doe_device_timestamp(uint64_t *dst, doe_stream_t stream);
int doe_device_timestamp_hz(int64_t *hz);
int doe_graph_capture_begin(doe_stream_t stream);
int doe_graph_capture_end(doe_stream_t stream, doe_graph_t *graph);
int doe_graph_launch(doe_graph_t graph, doe_stream_t stream);
int doe_graph_destroy(doe_graph_t graph);

/* ---- Q4_K_M quantized weights ----------------------------------------------
 * Block: 256 weights in 144 bytes -- f16 d, f16 dmin, 12 bytes of packed
 * 6-bit scales/mins, 128 bytes of nibbles (bench/tools/doppler_rdrr_q4k.py:
 * 11-15, 56-101).  A weight matrix [n][k] is row-wise: ceil(k/256) blocks
 * per row, row stride ceil(k/256)*144 bytes, values past k in the last block
 * ignored (doppler_rdrr_q4k.py:128-156).  The pointer must be 16-byte aligned.
 */

/* Dequantize to f32 out[n][k]; bit-exact RN_f32(d*sc*q - dmin*m).
 * Replaces the `dequant` op (runtime/zig/src/doe_wgsl/emit_csl_exec_v1.zig:
 * 164, pattern emitted by emit_csl_dequant.zig) with the canonical block
 * decode of doppler_rdrr_q4k.py:79-101. */
int doe_q4k_dequant(const void *weight_q4k, float *out, int64_t n, int64_t k,
                    doe_stream_t stream);

/* Decode GEMV output[i] = sum_k dequant(weight)[i,k] * activation[k], f32.
 * Replaces the `matmul_q4k` op (emit_csl_exec_v1.zig:162 -> pattern
 * fused_gemv_dequant, runtime/zig/src/doe_wgsl/emit_csl_fused.zig:47-200,
 * exported symbols activation/weight/output) and the reference interpreter's
 * fused_gemv (runtime/zig/src/tsir/reference_interpreter.zig:169-394).
 * activation: f32[k], output: f32[n]; k <= 65536 (past 16384 the K ranges
 * add into output atomically: the f32 summation order varies run to run). */
int doe_q4k_gemv(const void *weight_q4k, const float *activation, float *output,
                 int64_t n, int64_t k, doe_stream_t stream);

/* Q8_0 GEMV: output[i] = sum_k dequant(W)[i][k] * activation[k] (+
 * residual[i] when residual != NULL; residual == output is allowed).  W is
 * row-wise Q8_0: each row ceil(k / 32) blocks of 34 bytes, an f16 scale d then
 * 32 int8 quants q, weight = d * q (the block of
 * runtime/zig/src/doe_wgsl/csl_spec.zig:122-152, Q8_0_BLOCK_BYTES = 34; the
 * `q8_0` matmul quant format of emit_csl_host.zig:62 / emit_csl_exec_v1.zig:
 * 279-284; RDRR dtype "Q8_0", blockSizeElements 32, blockSizeBytes 34,
 * bench/tools/run_doe_csl_int4ple_transcript.py:1532-1565), the tail block
 * zero padded.  Replaces the decode `matmul` step at M = 1 when the model's
 * quantFormat is q8_0.  Weights 4-byte aligned (rows and blocks are only
 * 2-byte aligned), k <= 32768, f32 accumulation. */
int doe_q8_0_gemv(const void *weight_q8_0, const float *activation, float *output, int64_t n,
                  int64_t k, const float *residual, doe_stream_t stream);
/* doe_q8_0_gemv of rmsnorm(activation): activation * 1/sqrt(mean(a^2) +
 * norm_eps) * (norm_weight, or 1 + norm_weight when norm_weight_offset) --
 * the `input_norm` / `post_attn_norm` step before q/k/v_proj or gate/up_proj
 * (rmsnorm.wgsl; reference_interpreter.zig:510-526) folded into the GEMV. */
int doe_q8_0_gemv_norm(const void *weight_q8_0, const float *activation, float *output, int64_t n,
                       int64_t k, const float *norm_weight, float norm_eps, int norm_weight_offset,
                       const float *residual, doe_stream_t stream);
/* doe_q8_0_gemv whose activation is the combine of the split-attention
 * partials written by doe_attn_decode_partials (batch 1, k = num_heads x
 * head_dim, 1..8 splits; the combine formula is given there): the attention
 * combine + o_proj + attn_residual steps of a Q8_0 decode step in one
 * dispatch, reading the caller's partials buffer (no library workspace).
 * In every Q8_0 entry point only the residual may alias the output. */
int doe_q8_0_gemv_attn_out(const void *weight_q8_0, const float *attn_partials, int64_t splits,
                           int64_t num_heads, int64_t head_dim, float *output, int64_t n,
                           const float *residual, doe_stream_t stream);

/* doe_q8_0_gemv with the steps around a decode projection folded in, as
 * doe_q4k_gemv_fused: norm_weight != NULL runs the activation through
 * RMSNorm (the input_norm / post_attn_norm step); residual != NULL adds it
 * (residual == output allowed); gated != 0 takes rows as interleaved (gate,
 * up) pairs and writes n/2 values gelu_tanh(dot_2i) * dot_2i+1 (the
 * gate/up_proj -> activation steps; gelu_gated.wgsl:1-14).  gated and
 * residual are exclusive; gated needs n even. */
int doe_q8_0_gemv_fused(const void *weight_q8_0, const float *activation, float *output, int64_t n,
                        int64_t k, const float *norm_weight, float norm_eps, int norm_weight_offset,
                        const float *residual, int gated, doe_stream_t stream);
/* doe_q4k_gemv_qkv_rope_kv over Q8_0 rows: input_norm + q/k/v_proj + rope_q /
 * rope_k + the K/V cache write of a decode step in one dispatch, the q/k
 * rows of each head stored as interleaved rotation pairs (row 2i = dim i,
 * row 2i+1 = dim i + head_dim/2), the same arguments and rules. */
int doe_q8_0_gemv_qkv_rope_kv(const void *weight_q8_0, const float *activation, float *output,
                              int64_t hidden, const float *norm_weight, float norm_eps,
                              int norm_weight_offset, int64_t num_heads, int64_t num_kv_heads,
                              int64_t head_dim, const float *freq_cis, const int32_t *position_dev,
                              uint16_t *key_cache, uint16_t *val_cache, int64_t max_seq_len,
                              doe_stream_t stream);

/* Every form of the Q4_K decode GEMV in one call, plus two that chain GEMVs
 * without atomics (no reference counterpart: the reference's decode step
 * adds the residual in its own `residual` op, which the fused forms here
 * fold in):
 *   activation_parts: the activation is activation + parts[0] + ... +
 *     parts[activation_nparts - 1] (each k floats, 16-byte aligned, added in
 *     that order; at most 4 parts, k <= 8192); activation_sum, when
 *     non-NULL, receives that sum (the residual stream a later step reads).
 *   output_parts: the K reduction is split into ranges and range s stores
 *     its row sums to output_parts[s * n + row] (max_output_parts x n
 *     floats; the count used, 1..4, is returned in *output_nparts and
 *     depends only on n, k and the device), range 0 with the residual (if
 *     any) added; the GEMV result is their sum in range order, which the
 *     next GEMV forms by taking part 0 as its activation and the others as
 *     its activation_parts.  No norm or epilogue; the attention prologue may
 *     be used.
 *   residual_parts: the residual is residual + residual_parts[0] + ... +
 *     residual_parts[residual_nparts - 1] (each n floats, added in that
 *     order; at most 4, output apart from the residual, matrix-core kernel):
 *     a later GEMV takes the parts an earlier one added in its activation
 *     load and forms the same sum, where activation_sum would store it.
 * So a decode layer's residual adds happen in a fixed order: bit-identical
 * results on every run, where an in-place residual K split adds atomically.
 * The other fields are those of doe_q4k_gemv_fused (norm_weight, residual,
 * gated), doe_q4k_gemv_qkv_rope_kv (rope_kv != 0 with the head shape, rotary
 * table, device position and caches; n = (num_heads + 2 num_kv_heads) x
 * head_dim) and doe_q4k_gemv_attn_out (attn_partials != NULL with its
 * splits and head shape; activation NULL, k = num_heads x head_dim). */
typedef struct doe_q4k_gemv_args {
    const void *weight_q4k;
    const float *activation;
    const float *activation_parts;
    int64_t activation_nparts;
    float *activation_sum;
    float *output;
    int64_t n, k;
    const float *norm_weight;
    float norm_eps;
    int32_t norm_weight_offset;
    const float *residual;
    int32_t gated;
    int32_t rope_kv;
    int64_t num_heads, num_kv_heads, head_dim;
    const float *freq_cis;
    const int32_t *position_dev;
    uint16_t *key_cache, *val_cache;
    int64_t max_seq_len;
    const float *attn_partials;
    int64_t attn_splits, attn_num_heads, attn_head_dim;
    float *output_parts;
    int64_t max_output_parts;
    int32_t *output_nparts;
    const float *residual_parts;
    int64_t residual_nparts;
} doe_q4k_gemv_args;
int doe_q4k_gemv_ex(const doe_q4k_gemv_args *args, doe_stream_t stream);

/* The attention output projection of one sequence with the split-attention
 * combine folded into its activation load: output[i] = sum_k
 * dequant(W)[i][k] * attn[k] (+ residual[i]), attn = the combine of the
 * partials written by doe_attn_decode_partials (batch 1, num_heads x
 * head_dim = k, 1..8 splits).  Replaces the attention combine + o_proj +
 * attn_residual steps of a decode step.  residual == output (in place) may
 * split K over workgroups that add their partial sums atomically. */
int doe_q4k_gemv_attn_out(const void *weight_q4k, const float *attn_partials, int64_t splits,
                          int64_t num_heads, int64_t head_dim, float *output, int64_t n,
                          const float *residual, doe_stream_t stream);

/* Prefill GEMM c[m][n] = sum_k a[m][k] * dequant(b)[n][k]: a bf16 [m][k]
 * row-major, b row-wise Q4_K_M [n][k] (16-byte aligned), c f32 [m][n]
 * row-major.  Replaces the `matmul_q4k` op at M > 1 (pattern classified in
 * runtime/zig/src/doe_wgsl/emit_csl_classify.zig:287-297, lowered to SUMMA
 * with a dequantised B tile in emit_csl_matmul_q4k.zig:66-345).  Products
 * run on f16 matrix cores with f32 accumulation (a converted exactly to f16
 * with a per-row power-of-two scale, b dequantised to f16); rel-L2 against
 * the f32 reference ~2e-4.  Uses a library-owned workspace of m*ceil(k/64)*64*2
 * + 4m bytes, grown on demand (not during stream capture). */
int doe_q4k_gemm(const uint16_t *a_bf16, const void *b_q4k, float *c, int64_t m, int64_t n,
                 int64_t k, doe_stream_t stream);

/* doe_q4k_gemm with f32 activations a [m][k] (a prompt's f32 hidden states,
 * the step graphs' af32 activation format): each row is scaled by a power of
 * two and rounded once to f16 (11 significant bits) by the pre-pass, then
 * the same matrix-core GEMM; the same workspace rule. */
int doe_q4k_gemm_f32(const float *a, const void *b_q4k, float *c, int64_t m, int64_t n, int64_t k,
                     doe_stream_t stream);
/* The same GEMM over Q8_0 rows (the `matmul` op with quantFormat q8_0 at
 * M > 1, emit_csl_exec_v1.zig:279-284; block csl_spec.zig:121-153: 34 bytes
 * of f16 d and 32 int8 q, weight d * q, rows of ceil(k / 32) blocks, the
 * weight 4-byte aligned and under 2 GiB). */
int doe_q8_0_gemm_f32(const float *a, const void *b_q8_0, float *c, int64_t m, int64_t n, int64_t k,
                      doe_stream_t stream);
/* doe_q4k_gemm_f32 (weight_format 0) or doe_q8_0_gemm_f32 (1) with the
 * prefill steps around a projection folded in (gemma-3-270m-smoke.json:
 * 10-25): input_norm / post_attn_norm (norm_weight non-NULL: a's rows go
 * through RMSNorm, bit for bit the doe_rmsnorm op, before the f16 pre-pass),
 * attn_residual / ffn_residual (residual non-NULL: c = a W^T + residual,
 * residual may be c), or the GeGLU activation over the gate/up projection
 * (activation 1: columns (2j, 2j + 1) as doe_geglu_pairs; 2: columns (j, j +
 * n/2) as doe_geglu_halves; c is then [m][n/2]).  A residual and an
 * activation are exclusive; a and norm_weight must not alias c.  Each fused
 * result equals the unfused op sequence bit for bit. */
int doe_quant_gemm_f32_fused(const float *a, const void *b, float *c, int64_t m, int64_t n, int64_t k,
                             int weight_format, const float *norm_weight, float norm_eps, int norm_weight_offset,
                             const float *residual, int activation, doe_stream_t stream);

/* Symmetric int4 group-32 GEMV, batch m in 1..8: y[b][i] = sum_k
 * (q[i][k] - 8) * s[i][k/32] * x[b][k].  w_u4: eight nibbles per u32, element
 * k of row i at bits 4*(k%8) of word (i*k_dim + k)/8; scales f16 [n][k/32];
 * x f32 [m][k]; y f32 [m][n]; k a multiple of 256; 16-byte aligned.
 * Replaces the fused int4 dequant GEMV of
 * bench/kernels/compilation-corpus/complex_fused_gemv_dequant.wgsl:18-66
 * (bindings quant_weights, scales, input_vec, output; uniforms rows, cols,
 * group_size = 32), with f16 scales and an activation batch.  f16 matrix
 * cores, x split into two f16 halves (21+ bits), f32 accumulation; y is the
 * same bit for bit on every call (K ranges added in a fixed order).  x must
 * not alias y.  Uses library-owned workspaces (split-K partials and per-row-
 * block counts), grown on demand (not during stream capture); calls that
 * overlap on two streams share them. */
int doe_int4g32_gemv(const uint32_t *w_u4, const uint16_t *scales_f16, const float *x, float *y,
                     int64_t m, int64_t n, int64_t k, doe_stream_t stream);

/* Fused decode GEMV: the plain Q4_K GEMV with the neighbouring steps of the
 * Doppler decode step list folded in (runtime/zig/examples/execution-v1/
 * gemma-3-270m-smoke.json: input_norm -> q/k/v_proj, o_proj ->
 * attn_residual, post_attn_norm -> gate/up_proj -> activation, down_proj ->
 * ffn_residual; the reference's own fused_ffn pattern,
 * runtime/zig/src/doe_wgsl/emit_csl_fused_ffn.zig, fuses gate/up + activation).
 *   norm_weight != NULL: activation <- rmsnorm(activation) with eps
 *     norm_eps, weight w (norm_weight_offset 0) or 1 + w (1), as
 *     bench/inference-pipeline/kernels/rmsnorm.wgsl:15-93.
 *   residual != NULL: output[i] = dot_i + residual[i] (residual.wgsl).
 *     residual == output (in place) may split K over workgroups that add
 *     their partial sums atomically: the f32 addition order then varies.
 *   gated != 0: rows come as interleaved (gate, up) pairs; output has n/2
 *     values gelu_tanh(dot_2i) * dot_2i+1 (gelu_gated.wgsl:1-14).
 * gated and residual are exclusive; gated needs n even. */
int doe_q4k_gemv_fused(const void *weight_q4k, const float *activation, float *output,
                       int64_t n, int64_t k, const float *norm_weight, float norm_eps,
                       int norm_weight_offset, const float *residual, int gated,
                       doe_stream_t stream);

/* Fused q/k/v projection of one decode step: output = Wqkv . rmsnorm(x)
 * (rows [num_heads + 2 num_kv_heads][head_dim]), then RoPE on the q and k
 * rows and the f16 write of k, v into the caches [kv_heads][max_seq][head_dim]
 * at *position_dev -- the reference steps input_norm, q/k/v_proj, rope_q,
 * rope_k and the cache write of attention (execution-v1
 * gemma-3-270m-smoke.json decode steps; rope.wgsl; run_csl_webgpu_emulator.mjs:
 * 615-644) in one dispatch.  Within each q/k head the weight rows are
 * interleaved rotation pairs: row 2i holds dim i and row 2i+1 dim
 * i + head_dim/2 of the rotate-half form (a row permutation applied at load
 * time; q . k is unchanged because q and k share it, and k is cached in the
 * same order).  norm_weight may be NULL (no norm).  freq_cis holds
 * max_seq_len positions; a position outside [0, max_seq_len) leaves q/k
 * unrotated and writes no cache row.  num_kv_heads 0 projects and rotates the
 * q rows only (a shared-KV layer, whose attention reads an earlier layer's
 * cache: numKvSharedLayers, emit_csl_exec_v1.zig:720-723); the caches may
 * then be NULL. */
int doe_q4k_gemv_qkv_rope_kv(const void *weight_q4k, const float *activation, float *output,
                             int64_t hidden, const float *norm_weight, float norm_eps,
                             int norm_weight_offset, int64_t num_heads, int64_t num_kv_heads,
                             int64_t head_dim, const float *freq_cis,
                             const int32_t *position_dev, uint16_t *key_cache,
                             uint16_t *val_cache, int64_t max_seq_len, doe_stream_t stream);

/* Causal GQA prefill attention (flash form): out[i][h][:] = softmax over keys
 * j (j <= start_pos + i when causal) of q[i][h] . k[h/(Hq/Hkv)][j] * scale,
 * weighting v.  q bf16 [q_len][num_heads][128], k/v bf16
 * [num_kv_heads][kv_stride][128] (cache layout [kv_head][pos][dim]; keys
 * [0, kv_len) used), out f32 (out_bf16 = 0) or bf16 [q_len][num_heads][128];
 * all 16-byte aligned.  Replaces the tiled/causal path of the `attention` op
 * (attention_head256_f16kv.wgsl:72-267 with is_causal, query blocks of 32;
 * CPU tiled online softmax run_csl_webgpu_emulator.mjs:646-720).  Q.K^T on
 * bf16 matrix cores, P.V on f16 matrix cores (V converted exactly for |v| in
 * [2^-14, 65504]), f32 softmax and accumulation.  head_dim 128 only. */
int doe_attn_prefill(const uint16_t *q, const uint16_t *k, const uint16_t *v, void *out,
                     int out_bf16, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                     int64_t q_len, int64_t kv_len, int64_t kv_stride, int64_t start_pos,
                     float scale, int causal, doe_stream_t stream);

/* ---- attention ---------------------------------------------------------------
 * GQA decode attention over an f16 KV cache: one query token per sequence.
 * Replaces the `attention` op (emit_csl_exec_v1.zig:117 -> attention_decode;
 * Doppler kernel runtime/zig/tests/tsir/real/attention_head256_f16kv/
 * attention_head256_f16kv.wgsl: bindings Q (1), K (2), V (3), output (4),
 * kv_len_buffer (5); Uniforms num_heads, num_kv_heads, head_dim, seq_len,
 * scale, attn_softcap, sliding_window, kv_len_source, kv_layout, :14-38).
 *   q        [batch][num_heads][head_dim], f16 (q_f16 = 1) or f32
 *   k/v      f16; kv_layout 0: [batch][num_kv_heads][kv_stride][head_dim]
 *                  kv_layout 1: [batch][kv_stride][num_kv_heads][head_dim]
 *   out      [batch][num_heads][head_dim], f16 (out_f16 = 1) or f32
 *   kv_len   valid positions (0 <= kv_len <= kv_stride); when kv_len_dev is
 *            non-NULL the length is read from that device int32 instead
 *            (the reference's kv_len_buffer), so a captured graph can replay
 *            with a growing cache.
 *   the query sits at position kv_len - 1; sliding_window > 0 keeps keys
 *   [kv_len - sliding_window, kv_len); softcap > 0 applies tanh(s/cap)*cap.
 * head_dim 64/128/256/512, num_heads / num_kv_heads in {1, 2, 4, 8}.
 * q, k_cache and v_cache must be 16-byte aligned.
 * This entry point's kv_layout is the memory order; the reference's own
 * kv_layout uniform (contiguous / ring / paged positions) is taken by
 * doe_attention_dispatch below.
 * Uses a library-owned workspace for split-K partials: calls on one device
 * must not run concurrently on different streams. */
int doe_attn_decode(const void *q, int q_f16, const uint16_t *k_cache, const uint16_t *v_cache,
                    void *out, int out_f16, int64_t batch, int64_t num_heads,
                    int64_t num_kv_heads, int64_t head_dim, int64_t kv_len,
                    const int32_t *kv_len_dev, int64_t kv_stride, int kv_layout, float scale,
                    float softcap, int64_t sliding_window, doe_stream_t stream);

/* doe_attn_decode for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference, whose attention dispatch computes its
 * online softmax in one workgroup pass and so has no split partials.  Same
 * arguments, split choice and results as doe_attn_decode, but the split
 * partials live in a fixed 16 MiB device array per GPU (set up by doe_init;
 * DOE_E_NOT_INIT before that on the current device) instead of the library's
 * grow-only workspace: the call makes no hipMalloc / hipFree / synchronising
 * call.  Shapes whose partials exceed the array (batch x num_heads x splits x
 * (head_dim + 2) floats, 256-byte aligned halves) are rejected with
 * DOE_E_UNSUPPORTED.  Every call on one GPU shares that GPU's array: calls
 * that overlap in time on one GPU (different streams) race. */
int doe_attn_decode_noalloc(const void *q, int q_f16, const uint16_t *k_cache,
                            const uint16_t *v_cache, void *out, int out_f16, int64_t batch,
                            int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                            int64_t kv_len, const int32_t *kv_len_dev, int64_t kv_stride,
                            int kv_layout, float scale, float softcap, int64_t sliding_window,
                            doe_stream_t stream);

/* The reference attention dispatch itself: its Uniforms block field for
 * field (attention_head256_f16kv.wgsl:14-30) and its bindings Q (1), K (2),
 * V (3), output (4), kv_len_buffer (5), page_table (6), for any query_len
 * (:72-267; query i at absolute position start_pos + i).
 *   q        f32 [query_len][num_heads][head_dim]; output the same shape
 *   k/v      f16 [kv_capacity][num_kv_heads][head_dim] (the reference's order)
 *   keys     key_pos in [0, L), L = seq_len or kv_len_buffer[0]
 *            (kv_len_source 1); cache row of key_pos (:51-63): kv_start +
 *            key_pos; kv_layout 1 with sliding_window > 0: that modulo
 *            sliding_window (a ring); kv_layout 2: page_table[abs / page_size]
 *            * page_size + abs % page_size (page_table_len entries, clamped).
 *            Rows are clamped into [0, kv_capacity).
 *   visible  (:115-131) for query i, abs = start_pos + i: is_causal:
 *            key_pos <= abs - kv_start; sliding_window > 0 and abs >=
 *            sliding_window: key_pos >= abs - sliding_window + 1 - kv_start;
 *            scores scaled by scale, softcapped by attn_softcap; a query with
 *            no visible key writes zeros.
 * query_len 1 runs the split-K decode kernel; query_len > 1 an MFMA flash
 * kernel (16 queries x the query heads of one KV head per workgroup, f32 q
 * as f16 hi + lo, P in f16, f32 accumulation).  head_dim 64/128/256/512.
 * q, k and v must be 16-byte aligned. */
typedef struct {
    uint32_t num_heads, num_kv_heads, head_dim, seq_len, query_len;
    float scale;
    uint32_t is_causal, start_pos;
    float attn_softcap;
    uint32_t sliding_window, kv_len_source, kv_start, page_size, kv_layout, pad;
} doe_attention_uniforms;

int doe_attention_dispatch(const doe_attention_uniforms *u, const float *q, const uint16_t *k,
                           const uint16_t *v, float *output, const uint32_t *kv_len_buffer,
                           const uint32_t *page_table, int64_t page_table_len, int64_t kv_capacity,
                           doe_stream_t stream);

/* The multi-query form of the dispatch above over a decoder's cache: causal
 * attention of query_len prompt queries at positions start_pos + i over keys
 * [0, kv_len) of an f16 cache in either memory order (kv_layout 0
 * [num_kv_heads][kv_stride][head_dim], 1 [kv_stride][num_kv_heads]
 * [head_dim]), q f32 rows of q_row_stride floats ([num_heads][head_dim] at
 * the start of each row, e.g. the q part of a fused q/k/v projection),
 * output f32 rows of out_row_stride floats; sliding_window > 0 keeps the
 * last sliding_window keys of each query, softcap > 0 caps the scores.  The
 * prefill `attention` step of a step graph's prompt (gemma-3-270m-smoke.json
 * prefill; attention_head256_f16kv.wgsl:72-267 with is_causal).  A short
 * prompt splits its key blocks over the grid and merges the splits in a
 * second kernel, through a library-owned grow-only workspace (the workspace
 * rule of doe_attn_decode). */
int doe_attn_prefill_f16kv(const float *q, int64_t q_row_stride, const uint16_t *k_cache,
                           const uint16_t *v_cache, float *output, int64_t out_row_stride,
                           int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                           int64_t query_len, int64_t kv_len, int64_t kv_stride, int kv_layout,
                           int64_t start_pos, float scale, float softcap, int64_t sliding_window,
                           doe_stream_t stream);

/* The split-K half of doe_attn_decode without its combine: per query head
 * and split, the partial output o and (m, l) -- the running max of the
 * scores in log2 units and the sum of 2^(s - m) -- into the caller's
 * buffer: o [batch*num_heads][S][head_dim] f32, then ml
 * [batch*num_heads][S][2] f32 (partials_capacity floats in all).  S (at most
 * max_splits) is returned in *splits; it depends only on the shapes (the
 * cache length kv_stride when kv_len_dev is given), so a captured graph
 * keeps it.  The combine is done by the consumer (doe_q4k_gemv_attn_out):
 * out = sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), M = max_s m_s. */
int doe_attn_decode_partials(const void *q, int q_f16, const uint16_t *k_cache,
                             const uint16_t *v_cache, int64_t batch, int64_t num_heads,
                             int64_t num_kv_heads, int64_t head_dim, int64_t kv_len,
                             const int32_t *kv_len_dev, int64_t kv_stride, int kv_layout,
                             float scale, float softcap, int64_t sliding_window, float *partials,
                             int64_t partials_capacity, int64_t max_splits, int32_t *splits,
                             doe_stream_t stream);

/* ---- normalisation, position and elementwise ops ---------------------------
 * RMSNorm per row: out = x * 1/sqrt(mean(x^2) + eps) * (w or 1 + w).
 * Replaces the `rmsnorm` op (emit_csl_exec_v1.zig:128; rmsnorm.wgsl:1-93,
 * bindings input (1) weight (2) output (3), Uniforms size, eps). */
int doe_rmsnorm(const float *input, const float *weight, float *output, int64_t rows,
                int64_t size, float eps, int weight_offset, doe_stream_t stream);
/* RoPE, rotate-half pairs (i, i + D/2) in place on qk[seq][heads][head_dim]
 * with freq_cis[pos][D/2][2] = (cos, sin); pos = seq index + position_offset
 * (or + *position_dev when non-NULL).  Replaces the `rope` op (rope.wgsl:1-35:
 * bindings qk (1) freq_cis (2); Uniforms seq_len, head_dim, num_heads,
 * position_offset). */
int doe_rope(float *qk, const float *freq_cis, int64_t seq_len, int64_t num_heads,
             int64_t head_dim, int64_t position_offset, const int32_t *position_dev,
             doe_stream_t stream);
/* doe_rope over the first rotary_dim dims of each head only (rotate-half
 * pairs (i, i + rotary_dim/2), the other dims unchanged; freq_cis
 * [pos][rotary_dim/2][2]).  Replaces the `rope_partial` kernel of
 * qwen-3-6-27b-smoke.json (partialRotaryFactor 0.25: 64 of 256 dims; its
 * text-only mropeSection positions reduce to this 1D rotation). */
int doe_rope_partial(float *qk, const float *freq_cis, int64_t seq_len, int64_t num_heads, int64_t head_dim,
                     int64_t rotary_dim, int64_t position_offset, const int32_t *position_dev,
                     doe_stream_t stream);
/* out = gelu_tanh(gate) * up (clamped inner, gelu_gated.wgsl:1-14). */
int doe_geglu(const float *gate, const float *up, float *output, int64_t n, doe_stream_t stream);
/* out = input + residual (residual.wgsl; run_csl_webgpu_emulator.mjs:482-489);
 * output may be input or residual (in place). */
int doe_residual_add(const float *input, const float *residual, float *output, int64_t n,
                     doe_stream_t stream);
/* The prompt form of doe_q4k_gemv_qkv_rope_kv's epilogue, over `tokens` rows
 * of row_stride floats of a fused [q; k; v] projection (q/k rows interleaved
 * rotation pairs): token t at position start_pos + t has its q and k pairs
 * rotated by freq_cis[pos] in place and its k and v rows written as f16 into
 * the caches [num_kv_heads][max_seq_len][head_dim] -- the prefill rope_q /
 * rope_k steps (rope.wgsl with seq_len = the prompt) and the cache write of
 * the prompt (run_csl_webgpu_emulator.mjs:615-644).  Positions must lie in
 * the cache; num_kv_heads 0 rotates q only. */
int doe_qkv_rope_kv_rows(float *qkv, int64_t tokens, int64_t row_stride, int64_t num_heads,
                         int64_t num_kv_heads, int64_t head_dim, const float *freq_cis,
                         int64_t start_pos, uint16_t *key_cache, uint16_t *val_cache,
                         int64_t max_seq_len, doe_stream_t stream);
/* doe_qkv_rope_kv_rows for projections in head order (rows [q heads | k heads
 * | v heads], each head_dim wide): the rotate-half pairs (i, i + head_dim/2)
 * of doe_rope, with the same arithmetic, for every prompt row; k and v rows
 * into the caches [num_kv_heads][max_seq_len][head_dim]. */
int doe_qkv_rope_half_kv_rows(float *qkv, int64_t tokens, int64_t row_stride, int64_t num_heads,
                              int64_t num_kv_heads, int64_t head_dim, const float *freq_cis,
                              int64_t start_pos, uint16_t *key_cache, uint16_t *val_cache,
                              int64_t max_seq_len, doe_stream_t stream);
/* GeGLU over rows of [gate (n) | up (n)] (the `activation` step of a prompt):
 * out[t][i] = gelu_tanh(gate[t][i]) * up[t][i], gelu_gated.wgsl per row. */
int doe_geglu_halves(const float *gate_up, float *output, int64_t rows, int64_t n,
                     doe_stream_t stream);
/* GeGLU over interleaved (gate, up) pairs: out[i] = gelu_tanh(gate_up[2i]) *
 * gate_up[2i + 1] (gelu_gated.wgsl:1-14; the activation step of a prompt
 * whose gate/up projection rows are interleaved). */
int doe_geglu_pairs(const float *gate_up, float *output, int64_t n, doe_stream_t stream);
/* Per-layer-embedding combine: out = (projected + gathered) * scale, one f32
 * add then one f32 multiply per element -- the `ple_modulate` step
 * (emit_csl_exec_v1.zig:167-172: the element_wise part of the PLE composite,
 * kernelKey ple_residual) that joins the projected, normalised per-layer
 * inputs with the gathered per-layer embedding rows. */
int doe_ple_modulate(const float *projected, const float *gathered, float *output, int64_t n,
                     float scale, doe_stream_t stream);
/* Greedy sample: token = argmax(logits), lowest index on ties (sample.wgsl:
 * 17-55, run_csl_webgpu_emulator.mjs:841-878).  workspace: >= 8192 device
 * bytes. */
int doe_argmax(const float *logits, int64_t n, int32_t *token, void *workspace,
               doe_stream_t stream);
/* cache[h][pos][:] = f16(proj[h][:]) for K and V (run_csl_webgpu_emulator.mjs:
 * 615-644); position from `position` or *position_dev; positions outside
 * the cache are rejected (host) or skipped (device value). */
int doe_kv_write(const float *key_proj, const float *val_proj, uint16_t *key_cache,
                 uint16_t *val_cache, int64_t num_kv_heads, int64_t max_seq_len,
                 int64_t head_dim, int64_t position, const int32_t *position_dev, int kv_layout,
                 doe_stream_t stream);
/* out[t][:] = scale * f32(table[ids[t]][:]), zeros for ids outside the table
 * (the `embed` op, run_csl_webgpu_emulator.mjs:528-551; gather.wgsl). */
int doe_embed_gather(const uint16_t *table_f16, const int32_t *ids, float *output,
                     int64_t n_ids, int64_t vocab, int64_t hidden, float scale,
                     doe_stream_t stream);
/* The interpreter's gather (reference_interpreter.zig:4143-4276): out[t][:] =
 * table[ids[t]][:], u32 ids, f32 table.  The reference rejects a run with an
 * id >= vocab; here such a row is zero-filled and, when bad_ids != NULL, the
 * device int *bad_ids (cleared by this call) counts those ids, so the caller
 * can reject the result (the Python mirror does). */
int doe_gather_f32(const uint32_t *ids, const float *table, float *output, int64_t n_ids,
                   int64_t vocab, int64_t hidden, int32_t *bad_ids, doe_stream_t stream);

/* ---- f16-weight GEMV (lm_head) -----------------------------------------------
 * c[n] = alpha * sum_k a[k] * f32(b[n][k]); b f16 row-major (transpose_b = 1).
 * Replaces lm_head_gemv.wgsl main / main_multicol (runtime/zig/tests/tsir/
 * real/lm_head_gemv/lm_head_gemv.wgsl:58-180: bindings A (1) B (2) C (3),
 * Uniforms M, N, K, alpha, transpose_b).  k % 8 == 0, k <= 8192. */
int doe_f16_gemv(const uint16_t *b_f16, const float *a, float *c, int64_t n, int64_t k,
                 float alpha, doe_stream_t stream);
/* The same GEMV with all of the shader's uniforms: c[r][j] = alpha *
 * sum_i a[r][i] * B(j, i) for r < m, B(j, i) = b[j*k + i] (transpose_b = 1,
 * [N][K]) or b[i*n + j] (transpose_b = 0, [K][N]), any k (lm_head_gemv.wgsl
 * :105-143; main reads activation row 0, i.e. m = 1).  m = 1 against [N][K]
 * with k % 8 == 0, k <= 8192 and 16-byte aligned a and b runs the
 * doe_f16_gemv kernel; other shapes read b ceil(m / 8) times (ceil(m / 4)
 * for m <= 4).  m <= 524280, k <= 2^30. */
int doe_lm_head_gemv(const float *a, const uint16_t *b_f16, float *c, int64_t m, int64_t n,
                     int64_t k, float alpha, int transpose_b, doe_stream_t stream);
/* The lm_head with the final norm and the greedy sample folded in: a =
 * rmsnorm(a) when norm_weight != NULL; logits written when non-NULL; every
 * workgroup writes its best argmax key (see doe_decode_advance) to
 * argmax_partials (>= 1024 entries), *num_partials = workgroups used.
 * Replaces the final rmsnorm + lm_head + `sample` steps of a decode step. */
int doe_f16_gemv_argmax(const uint16_t *b_f16, const float *a, float *logits, int64_t n,
                        int64_t k, float alpha, const float *norm_weight, float norm_eps,
                        int norm_weight_offset, uint64_t *argmax_partials,
                        int64_t partials_capacity, int32_t *num_partials, doe_stream_t stream);

/* ---- Qwen 3.6 graph ops: gated activations and the gated-DeltaNet body ------
 * The ops of runtime/zig/examples/execution-v1/qwen-3-6-27b-smoke.json that
 * the attention path above does not cover, with the reference interpreter's
 * semantics (runtime/zig/src/tsir/reference_interpreter.zig).  f32 tensors,
 * caller-owned device buffers. */
/* output = act(gate) * input: kind 0 gelu (inner argument clamped to
 * [-15, 15]), 1 silu x / (1 + exp(z)), 2 sigmoid 1 / (1 + exp(z)), z =
 * clamp(-x, -15, 15).  Replaces the gelu_gated / silu_gated / sigmoid_gated
 * (o_gate) ops (tryGated, reference_interpreter.zig:954-1052: bindings gate,
 * input, output). */
int doe_gated(const float *gate, const float *input, float *output, int64_t n, int kind,
              doe_stream_t stream);
/* Per row of `hidden` values: output = input / sqrt(sum(input^2) + eps).
 * Replaces `l2_normalize` (tryL2Normalize, reference_interpreter.zig:
 * 1284-1361: bindings input, output; body hidden, eps). */
int doe_l2_normalize(const float *input, float *output, int64_t rows, int64_t hidden, float eps,
                     doe_stream_t stream);
/* Causal depthwise conv: input / output [tokens][channels], weight
 * [channels][kernel_size], bias [channels] or NULL; output[t][c] = bias[c]
 * + sum_k input[t - (kernel_size-1-k)][c] * weight[c][k] over the rows that
 * exist, rounded as the interpreter's f32 loop (bit for bit).  Replaces
 * `conv1d_depthwise` (tryConv1DDepthwise, reference_interpreter.zig:
 * 1363-1455: bindings input, weight, bias, output). */
int doe_conv1d_depthwise(const float *input, const float *weight, const float *bias, float *output,
                         int64_t tokens, int64_t channels, int64_t kernel_size, doe_stream_t stream);
/* Gated DeltaNet, single-query shared-norm form, over `tokens` tokens in
 * order: q, gate, output [tokens][heads][value_dim]; k, v
 * [tokens][heads][key_dim]; state [heads][value_dim][key_dim] updated in
 * place.  Per head alpha = 1 - exp(-a_log[h]) (a_log NULL: 0.5, the
 * interpreter's value); per state row d: dot = S[d] . k, S[d] = (1 - alpha)
 * S[d] + alpha (q[d] - dot) k, output[d] = S[d] . v + sigmoid(gate[d]) q[d].
 * key_dim <= 256.  Replaces `linear_attention` (tryLinearAttention,
 * reference_interpreter.zig:1457-1596; emit_kernel_body_linear_attention.zig:
 * bindings query, key, value, gate, linear_state, output). */
int doe_linear_attention(const float *q, const float *k, const float *v, const float *gate, float *state,
                         float *output, int64_t tokens, int64_t heads, int64_t key_dim, int64_t value_dim,
                         const float *a_log, doe_stream_t stream);

/* ---- synthetic inputs and decode-loop bookkeeping -----------------------------
 * No reference counterpart: the reference's decode numbers come from real
 * model weights (Doppler RDRR shards); benchmarks here run on seeded random
 * weights of the same shapes, drawn on the device.  Element i of a tensor
 * with seed s is a pure function of (s, i), so tensors are reproducible.
 * Q4_K blocks get d = f16(|N(0, d_sigma)|), dmin = f16(|N(0, dmin_sigma)|),
 * uniform 6-bit scales/mins and uniform nibbles. */
int doe_fill_normal_f16(uint16_t *out, int64_t n, uint64_t seed, float mean, float sigma,
                        doe_stream_t stream);
int doe_fill_normal_f32(float *out, int64_t n, uint64_t seed, float mean, float sigma,
                        doe_stream_t stream);
int doe_fill_uniform_i32(int32_t *out, int64_t n, uint64_t seed, int32_t lo, int32_t hi,
                         doe_stream_t stream);
int doe_fill_random_q4k(void *weight_q4k, int64_t nblocks, uint64_t seed, float d_sigma,
                        float dmin_sigma, doe_stream_t stream);
/* Q8_0 blocks: f16 scale |N(0, d_sigma)|, 32 uniform int8 quants. */
int doe_fill_random_q8_0(void *weight_q8_0, int64_t nblocks, uint64_t seed, float d_sigma,
                         doe_stream_t stream);
/* *checksum = XOR of the nbytes / 4 little-endian 32-bit words of buf
 * (nbytes a multiple of 16, buf 16-byte aligned), read once as a plain
 * stream by `workgroups` workgroups of 256 threads (0: automatic).  Used to
 * measure the read bandwidth the HBM-bound kernels are held against; no
 * reference counterpart. */
int doe_read_xor_u32(const void *buf, int64_t nbytes, uint32_t *checksum, int32_t workgroups,
                     doe_stream_t stream);
/* After a decode step, on the device: state = {pos, kv_len, prompt_len,
 * token}; pos += 1, kv_len = pos + 1, and the next token is ids[pos] inside
 * the prompt or the sampled *token (also stored to ids[pos]) after it.  With
 * argmax_partials (from doe_f16_gemv_argmax) the sampled token is first
 * reduced from them and stored to *token.  Keeps
 * a captured step graph replayable with no host round trip (the reference
 * reads back per token, bench/fixtures/r3-2-27b-doppler-frozen-af16/
 * reference-report.json:75 readbackInterval). */
int doe_decode_advance(int32_t *state, int32_t *token, int32_t *ids, int64_t max_seq,
                       const uint64_t *argmax_partials, int32_t num_partials,
                       doe_stream_t stream);

/* ---- tuning ----------------------------------------------------------------
 * Overrides a kernel launch-shape choice (0 restores the automatic choice).
 * Keys: "q4k_gemv.rowslots", "q4k_gemv.rows", "q4k_gemv.stream" (v > 0: the
 * streaming GEMV walking v row groups per workgroup, -1: never streaming),
 * "q4k_gemv.stream_depth" (2, 3, 4 or 6 units in flight per wave),
 * "int4_gemv.kernel" (1 one-shot, 2 streaming), "int4_gemv.depth" (2 or 3),
 * "int4_gemv.xcd" (1: workgroup ids in plain order, not a row block's K
 * ranges grouped on one XCD), "q8_0_gemv.rows" (1, 2 or 4 rows per wave group), "q8_0_gemv.depth" (1 or
 * 2 blocks loaded ahead), "attn_mq.splits" (1..16 key splits of the
 * multi-query attention), "attn_decode.splits",
 * "attn_decode.waves" (4: narrow workgroups; 8 or 16: the wide short-context
 * workgroup where the head shape allows it), "attn_decode.combine" (1: the
 * block-reduction split combine instead of the one-wave-per-column form),
 * "q4k_gemv.ksplit" (1: no K split over workgroups; 2-4: at least that many
 * K ranges where output parts are written), "q4k_gemv.forms" (bit 1: the
 * q/k/v epilogue without its fetched-ahead rotation; bit 2: the
 * attention-prologue o_proj in its fewest K ranges).  No
 * reference counterpart:
 * the reference fixes workgroup shapes per WGSL override constant
 * (lm_head_gemv.wgsl:168-169 MULTICOL_* overrides). */
int doe_tune_set(const char *key, int value);

#ifdef __cplusplus
}
#endif

#endif /* DOE_MI355X_H */
