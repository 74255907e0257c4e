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
 * activation: f32[k] (16-byte aligned), output: f32[n]. */
int doe_q4k_gemv(const void *weight_q4k, const float *activation, float *output,
                 int64_t n, int64_t k, doe_stream_t stream);

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
 * head_dim 64/128/256/512, num_heads / num_kv_heads in {1, 2, 4, 8} (512: <= 2).
 * Uses a library-owned workspace for split-K partials: calls on one device
 * must not run concurrently on different streams. */
int doe_attn_decode(const void *q, int q_f16, const uint16_t *k_cache, const uint16_t *v_cache,
                    void *out, int out_f16, int64_t batch, int64_t num_heads,
                    int64_t num_kv_heads, int64_t head_dim, int64_t kv_len,
                    const int32_t *kv_len_dev, int64_t kv_stride, int kv_layout, float scale,
                    float softcap, int64_t sliding_window, doe_stream_t stream);

/* ---- tuning ----------------------------------------------------------------
 * Overrides a kernel launch-shape choice (0 restores the automatic choice).
 * Keys: "q4k_gemv.rowslots", "q4k_gemv.rows", "attn_decode.splits".  No
 * reference counterpart:
 * the reference fixes workgroup shapes per WGSL override constant
 * (lm_head_gemv.wgsl:168-169 MULTICOL_* overrides). */
int doe_tune_set(const char *key, int value);

#ifdef __cplusplus
}
#endif

#endif /* DOE_MI355X_H */
