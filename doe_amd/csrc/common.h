// common.h -- shared plumbing for the gfx950 kernels behind the doe_mi355x C ABI.
//
// Every entry point returns DOE_OK (0) or a negative DOE_E* status and records
// a thread-local message readable through doe_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/doe_mi355x.h"

namespace doe {

// Sets the thread-local error message; returns `status` for tail calls.
int set_error(int status, const char *fmt, ...);
// Clears the thread-local error message.
void clear_error();
// Maps a HIP error to DOE_E_HIP with the HIP error string and a context.
int hip_fail(hipError_t e, const char *what);
// Checks that the library was initialised on the calling thread's device.
int require_init();
// Keeps a library workspace that a larger one has replaced allocated until
// doe_shutdown: kernels still queued, and HIP graphs captured earlier, may
// hold its address and keep using it.
void retire_workspace(void *ptr);
// Fills bytes [dst, dst + bytes) with `value` on a stream with a kernel
// (capturable into a HIP graph; no memset node).  Returns a DOE status.
int fill_bytes_async(void *dst, int value, size_t bytes, hipStream_t st);
// The query_len > 1 form of doe_attention_dispatch (attn_mq.hip).
int attention_dispatch_mq(const doe_attention_uniforms *u, const float *q, const uint16_t *k, const uint16_t *v,
                          float *output, const uint32_t *kv_len_buffer, const uint32_t *page_table,
                          int64_t page_table_len, int64_t kv_capacity, doe_stream_t stream);
// Looks up the allocation-free attention scratch of `device` (current).
int attn_scratch_setup(int device);
// Tuning hooks of individual kernels (0 = automatic).
int attn_set_splits(int value);
int mq_set_splits(int value);
int attn_set_waves(int value);
int attn_set_combine(int value);
int gemm_set_f16_operands(int value);
int int4_set_kernel(int value);
int int4_set_depth(int value);
int int4_set_xcd(int value);
int q8_0_set_tune(const char *key, int value);  // "q8_0_gemv.rows" / ".depth"

}  // namespace doe

#define DOE_HIP_CHECK(expr)                                        \
    do {                                                           \
        hipError_t doe_e_ = (expr);                                \
        if (doe_e_ != hipSuccess) return doe::hip_fail(doe_e_, #expr); \
    } while (0)

// Launch-error check after a kernel launch (asynchronous faults surface at sync).
#define DOE_LAUNCH_CHECK(name)                                        \
    do {                                                              \
        hipError_t doe_e_ = hipGetLastError();                        \
        if (doe_e_ != hipSuccess) return doe::hip_fail(doe_e_, name); \
    } while (0)

#define DOE_REQUIRE(cond, status, ...)                            \
    do {                                                          \
        if (!(cond)) return doe::set_error((status), __VA_ARGS__); \
    } while (0)

// Q4_K_M block constants (256 weights in 144 bytes).
#define DOE_Q4K_BLOCK_BYTES 144
#define DOE_Q4K_BLOCK_ELEMS 256

// gelu_tanh with the reference's clamp of the tanh argument
// (gelu_gated.wgsl:5-8, reference_interpreter.zig:1027-1045).
__device__ __forceinline__ float doe_gelu_tanh_clamped(float x) {
    float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    inner = fminf(fmaxf(inner, -15.0f), 15.0f);
    return 0.5f * x * (1.0f + tanhf(inner));
}

__device__ __forceinline__ float doe_half_bits_to_float(uint32_t bits16) {
    return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xffffu)));
}

// Epilogue of a fused q/k/v decode projection whose q and k rows come as
// interleaved rotation pairs (row 2i = dim i, row 2i+1 = dim i + head_dim/2 of
// the rotate-half form, rope.wgsl:1-35): the pair (row, row + 1) of finished
// sums is rotated by freq_cis[pos][i] (q and k rows), stored to y, and k and v
// rows are also written as f16 into the caches [kv_heads][max_seq][head_dim]
// at pos (read on the device).  A position outside [0, max_seq) leaves the
// rows unrotated and writes no cache row.
struct DoeRopeKv {
    const float *freq_cis;
    const int32_t *pos_dev;
    _Float16 *k_cache, *v_cache;
    int q_rows, kv_rows, head_dim, max_seq;
};

// The rotation of one row pair fetched ahead of its sums: the position and,
// for q / k rows at a position inside the cache, the pair's cos / sin.
struct DoeRopeAhead {
    int pos;
    float c, sn;
    bool rot;
};

// The position as a scalar load (one value for the wave, waited for on the
// scalar counter, so vector loads issued after it are not held back).
__device__ __forceinline__ int doe_rope_pos_scalar(const int32_t *pos_dev) {
    return *(const __attribute__((address_space(4))) int32_t *)pos_dev;
}

__device__ __forceinline__ void doe_rope_kv_pair_ahead(const DoeRopeKv &rk, const DoeRopeAhead &ra, int row,
                                                       float s0, float s1, float *y) {
#pragma clang fp contract(off)
    float r0 = s0, r1 = s1;
    if (ra.rot) {
        r0 = s0 * ra.c - s1 * ra.sn;
        r1 = s0 * ra.sn + s1 * ra.c;
    }
    y[row] = r0;
    y[row + 1] = r1;
    if (row >= rk.q_rows && ra.pos >= 0 && ra.pos < rk.max_seq) {
        const int kvr = row - rk.q_rows;
        const bool is_v = kvr >= rk.kv_rows;
        const int rr = is_v ? kvr - rk.kv_rows : kvr;
        const int h = rr / rk.head_dim;
        _Float16 *cache = is_v ? rk.v_cache : rk.k_cache;
        const size_t ci = ((size_t)h * rk.max_seq + ra.pos) * rk.head_dim + row % rk.head_dim;
        cache[ci] = (_Float16)r0;
        cache[ci + 1] = (_Float16)r1;
    }
}

__device__ __forceinline__ void doe_rope_kv_pair(const DoeRopeKv &rk, int row, float s0, float s1, float *y) {
    const int pos = rk.pos_dev[0];
    DoeRopeAhead ra{pos, 1.0f, 0.0f, false};
    if (pos >= 0 && pos < rk.max_seq && row < rk.q_rows + rk.kv_rows) {  // freq_cis holds max_seq positions
        const int i = (row % rk.head_dim) >> 1, half = rk.head_dim >> 1;
        ra.c = rk.freq_cis[((size_t)pos * half + i) * 2];
        ra.sn = rk.freq_cis[((size_t)pos * half + i) * 2 + 1];
        ra.rot = true;
    }
    doe_rope_kv_pair_ahead(rk, ra, row, s0, s1, y);
}
