// elementwise.hip -- RMSNorm, RoPE, GeGLU, residual add, argmax, KV write and
// embedding gather for gfx950.  These are the small ops around the decode
// GEMVs; each is HBM- or latency-bound and written for one pass over its data.
#include "common.h"

#include <math.h>

namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sum over a workgroup of `nwaves` waves through LDS (result in every thread).
__device__ __forceinline__ float block_sum(float v, float *sh, int nwaves) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < nwaves; ++w) t += sh[w];
    __syncthreads();
    return t;
}

// RMSNorm, one workgroup per row (rmsnorm.wgsl:15-53 / :55-93; the
// interpreter's numerics, reference_interpreter.zig:510-526, are an f32 sum of
// squares, mean = sum / H, inv = 1 / sqrt(mean + eps), out = x * inv * w).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x,
                                                      const float *__restrict__ w,
                                                      float *__restrict__ out, int h, float eps,
                                                      int weight_offset) {
    __shared__ float sh[4];
    const float *xr = x + (size_t)blockIdx.x * h;
    float *orow = out + (size_t)blockIdx.x * h;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < h; i += 256) ss = fmaf(xr[i], xr[i], ss);
    ss = block_sum(ss, sh, 4);
    const float inv = 1.0f / sqrtf(ss / (float)h + eps);
    for (int i = threadIdx.x; i < h; i += 256) {
        const float scale = weight_offset ? 1.0f + w[i] : w[i];
        orow[i] = xr[i] * inv * scale;
    }
}

// RoPE, rotate-half pairs (i, i + D/2) (rope.wgsl:12-35).  Products and
// differences are rounded separately, as the reference's scalar code does.
// rot < head_dim: partial rotary (the rope_partial kernel of
// qwen-3-6-27b-smoke.json, partialRotaryFactor): pairs (i, i + rot/2) of each
// head's first rot dims, the others unchanged; freq_cis [pos][rot/2][2].
__global__ __launch_bounds__(256) void rope_kernel(float *__restrict__ qk,
                                                   const float *__restrict__ freq_cis, int seq_len,
                                                   int num_heads, int head_dim, int rot, int pos_off,
                                                   const int32_t *__restrict__ pos_dev) {
#pragma clang fp contract(off)
    const int half = rot >> 1;
    const long total = (long)seq_len * num_heads * half;
    const int base_pos = pos_dev ? pos_dev[0] : pos_off;
    for (long g = (long)blockIdx.x * 256 + threadIdx.x; g < total; g += (long)gridDim.x * 256) {
        const int i = (int)(g % half);
        const long sh = g / half;  // seq * num_heads + head
        const int s = (int)(sh / num_heads);
        const long pos = (long)s + base_pos;
        float *base = qk + sh * head_dim;
        const float x0 = base[i], x1 = base[i + half];
        const float c = freq_cis[(pos * half + i) * 2], sn = freq_cis[(pos * half + i) * 2 + 1];
        base[i] = x0 * c - x1 * sn;
        base[i + half] = x0 * sn + x1 * c;
    }
}

__global__ __launch_bounds__(256) void geglu_kernel(const float *__restrict__ gate,
                                                    const float *__restrict__ up,
                                                    float *__restrict__ out, long n) {
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256)
        out[i] = doe_gelu_tanh_clamped(gate[i]) * up[i];
}

// out may be a or b: each element is read before it is written
__global__ __launch_bounds__(256) void residual_kernel(const float *a, const float *b, float *out, long n) {
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256)
        out[i] = a[i] + b[i];
}

// Prompt rows of a fused [q; k; v] projection whose q and k rows are
// interleaved rotation pairs (row 2i = dim i, 2i + 1 = dim i + D/2 of the
// rotate-half form): token t (position start_pos + t) has its q/k pairs
// rotated by freq_cis[pos][i] and its k and v rows stored as f16 into the
// caches [kv_heads][max_seq][D] at pos -- the decode epilogue's arithmetic,
// one thread per row pair.
__global__ __launch_bounds__(256) void rope_kv_rows_kernel(float *qkv, long row_stride, int tokens, int q_rows,
                                                           int kv_rows, int head_dim, const float *__restrict__ freq,
                                                           int start_pos, _Float16 *kc, _Float16 *vc, int max_seq) {
#pragma clang fp contract(off)
    const int npairs = (q_rows + 2 * kv_rows) >> 1;
    const long total = (long)tokens * npairs;
    for (long gi = (long)blockIdx.x * 256 + threadIdx.x; gi < total; gi += (long)gridDim.x * 256) {
        const int t = (int)(gi / npairs), row = 2 * (int)(gi % npairs);
        const int pos = start_pos + t;
        float *r = qkv + (size_t)t * row_stride;
        const float s0 = r[row], s1 = r[row + 1];
        float r0 = s0, r1 = s1;
        const int dim = row % head_dim;
        if (row < q_rows + kv_rows) {
            const int i = dim >> 1, half = head_dim >> 1;
            const float c = freq[((size_t)pos * half + i) * 2], sn = freq[((size_t)pos * half + i) * 2 + 1];
            r0 = s0 * c - s1 * sn;
            r1 = s0 * sn + s1 * c;
            r[row] = r0;
            r[row + 1] = r1;
        }
        if (row >= q_rows) {
            const int kvr = row - q_rows;
            const bool is_v = kvr >= kv_rows;
            const int h = (is_v ? kvr - kv_rows : kvr) / head_dim;
            _Float16 *cache = is_v ? vc : kc;
            const size_t ci = ((size_t)h * max_seq + pos) * head_dim + dim;
            cache[ci] = (_Float16)r0;
            cache[ci + 1] = (_Float16)r1;
        }
    }
}

// Rotate-half form of rope_kv_rows (the doe_rope pairing, i and i + D/2 of
// each head): q and k heads rotated in place, k and v rows into the caches.
__global__ __launch_bounds__(256) void rope_half_kv_rows_kernel(float *qkv, long row_stride, int tokens, int q_heads,
                                                                int kv_heads, int head_dim,
                                                                const float *__restrict__ freq, int start_pos,
                                                                _Float16 *kc, _Float16 *vc, int max_seq) {
#pragma clang fp contract(off)
    const int half = head_dim >> 1, heads = q_heads + 2 * kv_heads;
    const long total = (long)tokens * heads * half;
    for (long gi = (long)blockIdx.x * 256 + threadIdx.x; gi < total; gi += (long)gridDim.x * 256) {
        const int i = (int)(gi % half);
        const long th = gi / half;
        const int t = (int)(th / heads), hh = (int)(th % heads);
        const int pos = start_pos + t;
        float *base = qkv + (size_t)t * row_stride + (size_t)hh * head_dim;
        const float x0 = base[i], x1 = base[i + half];
        float r0 = x0, r1 = x1;
        if (hh < q_heads + kv_heads) {
            const float c = freq[((size_t)pos * half + i) * 2], sn = freq[((size_t)pos * half + i) * 2 + 1];
            r0 = x0 * c - x1 * sn;
            r1 = x0 * sn + x1 * c;
            base[i] = r0;
            base[i + half] = r1;
        }
        if (hh >= q_heads) {
            const bool is_v = hh >= q_heads + kv_heads;
            const int h = is_v ? hh - q_heads - kv_heads : hh - q_heads;
            _Float16 *cache = is_v ? vc : kc;
            const size_t ci = ((size_t)h * max_seq + pos) * head_dim + i;
            cache[ci] = (_Float16)r0;
            cache[ci + half] = (_Float16)r1;
        }
    }
}

// GeGLU over rows of [gate (n) | up (n)]: out[t][i] = gelu(gu[t][i]) * gu[t][n + i]
__global__ __launch_bounds__(256) void geglu_halves_kernel(const float *__restrict__ gu, float *__restrict__ out,
                                                           int rows, int n) {
    const long total = (long)rows * n;
    for (long g = (long)blockIdx.x * 256 + threadIdx.x; g < total; g += (long)gridDim.x * 256) {
        const long t = g / n, i = g % n;
        out[g] = doe_gelu_tanh_clamped(gu[t * 2 * n + i]) * gu[t * 2 * n + n + i];
    }
}

// GeGLU over interleaved (gate, up) columns: out[i] = gelu(gu[2i]) * gu[2i+1]
__global__ __launch_bounds__(256) void geglu_pairs_kernel(const float2 *__restrict__ gu, float *__restrict__ out,
                                                          long n) {
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        const float2 p = gu[i];
        out[i] = doe_gelu_tanh_clamped(p.x) * p.y;
    }
}

// (projected + gathered) * scale: one f32 add, then one f32 multiply (no fma)
__global__ __launch_bounds__(256) void ple_modulate_kernel(const float *__restrict__ a,
                                                           const float *__restrict__ b,
                                                           float *__restrict__ out, long n, float scale) {
#pragma clang fp contract(off)
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256)
        out[i] = (a[i] + b[i]) * scale;
}

// Argmax keys: ordered float bits in the high word, inverted index in the low
// word, so an unsigned max picks the largest value and, on a tie, the lowest
// index (run_csl_webgpu_emulator.mjs:841-878: strict '>' from -FLT_MAX, index
// 0).  NaN never wins (it fails every '>' in the reference).
__device__ __forceinline__ unsigned long long argmax_key(float v, unsigned idx) {
    if (v != v) return 0ull;
    unsigned u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (0xffffffffu - idx);
}

__device__ __forceinline__ unsigned long long max_u64(unsigned long long a, unsigned long long b) {
    return a > b ? a : b;
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *__restrict__ logits, long n,
                                                             unsigned long long *__restrict__ part) {
    __shared__ unsigned long long sh[4];
    unsigned long long best = 0;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256)
        best = max_u64(best, argmax_key(logits[i], (unsigned)i));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) best = max_u64(best, __shfl_xor(best, o, 64));
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = max_u64(max_u64(sh[0], sh[1]), max_u64(sh[2], sh[3]));
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const unsigned long long *__restrict__ part,
                                                           int nparts, int32_t *__restrict__ out) {
    __shared__ unsigned long long sh[4];
    // the reference's starting point: value -FLT_MAX at index 0
    unsigned long long best = argmax_key(-3.402823466e38f, 0u);
    for (int i = threadIdx.x; i < nparts; i += 256) best = max_u64(best, part[i]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) best = max_u64(best, __shfl_xor(best, o, 64));
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        best = max_u64(max_u64(sh[0], sh[1]), max_u64(sh[2], sh[3]));
        out[0] = (int32_t)(0xffffffffu - (unsigned)(best & 0xffffffffull));
    }
}

// KV write (run_csl_webgpu_emulator.mjs:615-644): cache[h][pos][:] =
// f16(proj[h][:]) (RNE).  A position outside the cache writes nothing.
__global__ __launch_bounds__(256) void kv_write_kernel(const float *__restrict__ kp,
                                                       const float *__restrict__ vp,
                                                       _Float16 *__restrict__ kc,
                                                       _Float16 *__restrict__ vc, int kvh,
                                                       int max_seq, int head_dim, int pos_host,
                                                       const int32_t *__restrict__ pos_dev,
                                                       int layout) {
    const int pos = pos_dev ? pos_dev[0] : pos_host;
    if (pos < 0 || pos >= max_seq) return;
    const int total = kvh * head_dim;
    for (int g = blockIdx.x * 256 + threadIdx.x; g < total; g += gridDim.x * 256) {
        const int h = g / head_dim, d = g % head_dim;
        const size_t dst = layout == 0 ? ((size_t)h * max_seq + pos) * head_dim + d
                                       : ((size_t)pos * kvh + h) * head_dim + d;
        kc[dst] = (_Float16)kp[g];
        vc[dst] = (_Float16)vp[g];
    }
}

// Embedding gather (run_csl_webgpu_emulator.mjs:528-551): out[t] =
// scale * f32(table[id[t]]), zeros for ids outside the table.
__global__ __launch_bounds__(256) void embed_kernel(const _Float16 *__restrict__ table,
                                                    const int32_t *__restrict__ ids,
                                                    float *__restrict__ out, int n_ids, int vocab,
                                                    int hidden, float scale) {
    const long total = (long)n_ids * hidden;
    for (long g = (long)blockIdx.x * 256 + threadIdx.x; g < total; g += (long)gridDim.x * 256) {
        const int t = (int)(g / hidden), d = (int)(g % hidden);
        const int id = ids[t];
        out[g] = (id >= 0 && id < vocab) ? (float)table[(size_t)id * hidden + d] * scale : 0.0f;
    }
}

// Strict f32 gather (reference_interpreter.zig:4143-4276): out[t] =
// table[ids[t]] for u32 ids; an id outside the table zero-fills its row and
// is counted in *bad (the interpreter rejects such a run).  VEC = 4 moves
// float4 runs when hidden % 4 == 0.
template <int VEC>
__global__ __launch_bounds__(256) void gather_f32_kernel(const uint32_t *__restrict__ ids,
                                                         const float *__restrict__ table,
                                                         float *__restrict__ out, int n_ids,
                                                         uint32_t vocab, int hidden, int *bad) {
    typedef float fv __attribute__((ext_vector_type(VEC)));
    const int per_row = hidden / VEC;
    const long total = (long)n_ids * per_row;
    for (long g = (long)blockIdx.x * 256 + threadIdx.x; g < total; g += (long)gridDim.x * 256) {
        const int t = (int)(g / per_row), d = (int)(g % per_row);
        const uint32_t id = ids[t];
        fv v = (fv)0.0f;
        if (id < vocab)
            v = *reinterpret_cast<const fv *>(table + (size_t)id * hidden + (size_t)d * VEC);
        else if (d == 0 && bad)
            atomicAdd(bad, 1);
        *reinterpret_cast<fv *>(out + (size_t)t * hidden + (size_t)d * VEC) = v;
    }
}

unsigned grid_for(long n, unsigned cap = 4096) {
    long b = (n + 255) / 256;
    if (b < 1) b = 1;
    return (unsigned)(b > cap ? cap : b);
}

}  // namespace

extern "C" {

int doe_rmsnorm(const float *input, const float *weight, float *output, int64_t rows, int64_t size,
                float eps, int weight_offset, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(rows >= 0 && size >= 0 && rows <= 0x7fffffff && size <= 0x7fffffff, DOE_E_INVALID,
                "bad rmsnorm shape");
    if (rows == 0 || size == 0) return DOE_OK;
    DOE_REQUIRE(input && weight && output, DOE_E_INVALID, "null pointer");
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream, input,
                       weight, output, (int)size, eps, weight_offset);
    DOE_LAUNCH_CHECK("rmsnorm_kernel");
    return DOE_OK;
}

int doe_rope(float *qk, const float *freq_cis, int64_t seq_len, int64_t num_heads, int64_t head_dim,
             int64_t position_offset, const int32_t *position_dev, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(seq_len >= 0 && num_heads >= 0 && head_dim > 0 && (head_dim % 2) == 0 &&
                    position_offset >= 0,
                DOE_E_INVALID, "bad rope shape");
    const long total = (long)seq_len * num_heads * (head_dim / 2);
    if (total == 0) return DOE_OK;
    DOE_REQUIRE(qk && freq_cis, DOE_E_INVALID, "null pointer");
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream, qk,
                       freq_cis, (int)seq_len, (int)num_heads, (int)head_dim, (int)head_dim, (int)position_offset,
                       position_dev);
    DOE_LAUNCH_CHECK("rope_kernel");
    return DOE_OK;
}

int doe_rope_partial(float *qk, const float *freq_cis, int64_t seq_len, int64_t num_heads, int64_t head_dim,
                     int64_t rotary_dim, int64_t position_offset, const int32_t *position_dev, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(seq_len >= 0 && num_heads >= 0 && head_dim > 0 && rotary_dim > 0 && (rotary_dim % 2) == 0 &&
                    rotary_dim <= head_dim && position_offset >= 0 && seq_len * num_heads * head_dim < (1L << 31),
                DOE_E_INVALID, "bad rope shape (rotary_dim %lld of head_dim %lld)", (long long)rotary_dim,
                (long long)head_dim);
    const long total = (long)seq_len * num_heads * (rotary_dim / 2);
    if (total == 0) return DOE_OK;
    DOE_REQUIRE(qk && freq_cis, DOE_E_INVALID, "null pointer");
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream, qk,
                       freq_cis, (int)seq_len, (int)num_heads, (int)head_dim, (int)rotary_dim, (int)position_offset,
                       position_dev);
    DOE_LAUNCH_CHECK("rope_kernel");
    return DOE_OK;
}

int doe_geglu(const float *gate, const float *up, float *output, int64_t n, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(n >= 0, DOE_E_INVALID, "negative size");
    if (n == 0) return DOE_OK;
    DOE_REQUIRE(gate && up && output, DOE_E_INVALID, "null pointer");
    hipLaunchKernelGGL(geglu_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, gate, up,
                       output, (long)n);
    DOE_LAUNCH_CHECK("geglu_kernel");
    return DOE_OK;
}

int doe_residual_add(const float *input, const float *residual, float *output, int64_t n,
                     doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(n >= 0, DOE_E_INVALID, "negative size");
    if (n == 0) return DOE_OK;
    DOE_REQUIRE(input && residual && output, DOE_E_INVALID, "null pointer");
    hipLaunchKernelGGL(residual_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, input,
                       residual, output, (long)n);
    DOE_LAUNCH_CHECK("residual_kernel");
    return DOE_OK;
}

int doe_qkv_rope_kv_rows(float *qkv, int64_t tokens, int64_t row_stride, int64_t num_heads, int64_t num_kv_heads,
                         int64_t head_dim, const float *freq_cis, int64_t start_pos, uint16_t *key_cache,
                         uint16_t *val_cache, int64_t max_seq_len, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(tokens >= 0 && num_heads > 0 && num_kv_heads >= 0 && head_dim > 0 && (head_dim % 2) == 0 &&
                    start_pos >= 0 && max_seq_len > 0 && start_pos + tokens <= max_seq_len &&
                    row_stride >= (num_heads + 2 * num_kv_heads) * head_dim && max_seq_len < (1 << 30),
                DOE_E_INVALID, "bad prompt q/k/v shape (positions %lld..%lld in a %lld-row cache)",
                (long long)start_pos, (long long)(start_pos + tokens - 1), (long long)max_seq_len);
    if (tokens == 0) return DOE_OK;
    DOE_REQUIRE(qkv && freq_cis && (num_kv_heads == 0 || (key_cache && val_cache)), DOE_E_INVALID, "null pointer");
    const long total = (long)tokens * ((num_heads + 2 * num_kv_heads) * head_dim / 2);
    hipLaunchKernelGGL(rope_kv_rows_kernel, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream, qkv,
                       (long)row_stride, (int)tokens, (int)(num_heads * head_dim), (int)(num_kv_heads * head_dim),
                       (int)head_dim, freq_cis, (int)start_pos, (_Float16 *)key_cache, (_Float16 *)val_cache,
                       (int)max_seq_len);
    DOE_LAUNCH_CHECK("rope_kv_rows_kernel");
    return DOE_OK;
}

int doe_qkv_rope_half_kv_rows(float *qkv, int64_t tokens, int64_t row_stride, int64_t num_heads,
                              int64_t num_kv_heads, int64_t head_dim, const float *freq_cis, int64_t start_pos,
                              uint16_t *key_cache, uint16_t *val_cache, int64_t max_seq_len, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(tokens >= 0 && num_heads >= 0 && num_kv_heads >= 0 && head_dim > 0 && (head_dim % 2) == 0 &&
                    start_pos >= 0 && max_seq_len > 0,
                DOE_E_INVALID, "bad rope rows shape");
    DOE_REQUIRE(row_stride >= (num_heads + 2 * num_kv_heads) * head_dim, DOE_E_INVALID,
                "row_stride %lld shorter than the q/k/v rows", (long long)row_stride);
    DOE_REQUIRE(start_pos + tokens <= max_seq_len, DOE_E_INVALID, "positions %lld..%lld outside the %lld-row cache",
                (long long)start_pos, (long long)(start_pos + tokens - 1), (long long)max_seq_len);
    const long total = (long)tokens * (num_heads + 2 * num_kv_heads) * (head_dim / 2);
    if (total == 0) return DOE_OK;
    DOE_REQUIRE(qkv && freq_cis && (num_kv_heads == 0 || (key_cache && val_cache)), DOE_E_INVALID, "null pointer");
    hipLaunchKernelGGL(rope_half_kv_rows_kernel, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream, qkv,
                       (long)row_stride, (int)tokens, (int)num_heads, (int)num_kv_heads, (int)head_dim, freq_cis,
                       (int)start_pos, (_Float16 *)key_cache, (_Float16 *)val_cache, (int)max_seq_len);
    DOE_LAUNCH_CHECK("rope_half_kv_rows_kernel");
    return DOE_OK;
}

int doe_geglu_halves(const float *gate_up, float *output, int64_t rows, int64_t n, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(rows >= 0 && n >= 0 && n <= 0x3fffffff && rows <= 0x7fffffff, DOE_E_INVALID, "bad geglu shape");
    if (rows == 0 || n == 0) return DOE_OK;
    DOE_REQUIRE(gate_up && output, DOE_E_INVALID, "null pointer");
    hipLaunchKernelGGL(geglu_halves_kernel, dim3(grid_for(rows * n)), dim3(256), 0, (hipStream_t)stream, gate_up,
                       output, (int)rows, (int)n);
    DOE_LAUNCH_CHECK("geglu_halves_kernel");
    return DOE_OK;
}

int doe_geglu_pairs(const float *gate_up, float *output, int64_t n, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(n >= 0, DOE_E_INVALID, "negative size");
    if (n == 0) return DOE_OK;
    DOE_REQUIRE(gate_up && output && ((uintptr_t)gate_up & 7) == 0, DOE_E_INVALID,
                "null or misaligned pointer (gate_up 8-byte aligned)");
    hipLaunchKernelGGL(geglu_pairs_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                       (const float2 *)gate_up, output, (long)n);
    DOE_LAUNCH_CHECK("geglu_pairs_kernel");
    return DOE_OK;
}

int doe_ple_modulate(const float *projected, const float *gathered, float *output, int64_t n, float scale,
                     doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(n >= 0, DOE_E_INVALID, "negative size");
    if (n == 0) return DOE_OK;
    DOE_REQUIRE(projected && gathered && output, DOE_E_INVALID, "null pointer");
    hipLaunchKernelGGL(ple_modulate_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, projected,
                       gathered, output, (long)n, scale);
    DOE_LAUNCH_CHECK("ple_modulate_kernel");
    return DOE_OK;
}

int doe_argmax(const float *logits, int64_t n, int32_t *token, void *workspace,
               doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(n > 0 && n <= 0x7fffffff, DOE_E_INVALID, "argmax needs 0 < n < 2^31");
    DOE_REQUIRE(logits && token && workspace, DOE_E_INVALID, "null pointer");
    const unsigned parts = grid_for(n, 1024);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(parts), dim3(256), 0, (hipStream_t)stream, logits,
                       (long)n, (unsigned long long *)workspace);
    DOE_LAUNCH_CHECK("argmax_partial_kernel");
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream,
                       (const unsigned long long *)workspace, (int)parts, token);
    DOE_LAUNCH_CHECK("argmax_final_kernel");
    return DOE_OK;
}

int doe_kv_write(const float *key_proj, const float *val_proj, uint16_t *key_cache,
                 uint16_t *val_cache, int64_t num_kv_heads, int64_t max_seq_len, int64_t head_dim,
                 int64_t position, const int32_t *position_dev, int kv_layout,
                 doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(num_kv_heads >= 0 && head_dim >= 0 && max_seq_len > 0, DOE_E_INVALID,
                "bad kv_write shape");
    DOE_REQUIRE(kv_layout == 0 || kv_layout == 1, DOE_E_UNSUPPORTED, "kv_layout must be 0 or 1");
    DOE_REQUIRE(position_dev || (position >= 0 && position < max_seq_len), DOE_E_INVALID,
                "position %lld exceeds max_seq_len %lld", (long long)position, (long long)max_seq_len);
    const long total = (long)num_kv_heads * head_dim;
    if (total == 0) return DOE_OK;
    DOE_REQUIRE(key_proj && val_proj && key_cache && val_cache, DOE_E_INVALID, "null pointer");
    hipLaunchKernelGGL(kv_write_kernel, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream,
                       key_proj, val_proj, (_Float16 *)key_cache, (_Float16 *)val_cache,
                       (int)num_kv_heads, (int)max_seq_len, (int)head_dim, (int)position,
                       position_dev, kv_layout);
    DOE_LAUNCH_CHECK("kv_write_kernel");
    return DOE_OK;
}

int doe_gather_f32(const uint32_t *ids, const float *table, float *output, int64_t n_ids,
                   int64_t vocab, int64_t hidden, int32_t *bad_ids, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(n_ids >= 0 && vocab >= 0 && hidden >= 0 && vocab <= 0xffffffffL &&
                    n_ids <= 0x7fffffff && hidden <= 0x7fffffff,
                DOE_E_INVALID, "bad gather shape");
    hipStream_t st = (hipStream_t)stream;
    if (bad_ids) {
        DOE_REQUIRE(((uintptr_t)bad_ids & 3) == 0, DOE_E_INVALID, "bad_ids must be 4-byte aligned");
        rc = doe::fill_bytes_async(bad_ids, 0, 4, st);
        if (rc) return rc;
    }
    const long total = (long)n_ids * hidden;
    if (total == 0) return DOE_OK;
    DOE_REQUIRE(table || vocab == 0, DOE_E_INVALID, "null table");
    DOE_REQUIRE(ids && output, DOE_E_INVALID, "null pointer");
    const bool v4 = (hidden % 4) == 0 && ((uintptr_t)table & 15) == 0 && ((uintptr_t)output & 15) == 0;
    if (v4)
        hipLaunchKernelGGL(gather_f32_kernel<4>, dim3(grid_for(total / 4)), dim3(256), 0, st, ids, table,
                           output, (int)n_ids, (uint32_t)vocab, (int)hidden, (int *)bad_ids);
    else
        hipLaunchKernelGGL(gather_f32_kernel<1>, dim3(grid_for(total)), dim3(256), 0, st, ids, table,
                           output, (int)n_ids, (uint32_t)vocab, (int)hidden, (int *)bad_ids);
    DOE_LAUNCH_CHECK("gather_f32_kernel");
    return DOE_OK;
}

int doe_embed_gather(const uint16_t *table_f16, const int32_t *ids, float *output, int64_t n_ids,
                     int64_t vocab, int64_t hidden, float scale, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(n_ids >= 0 && vocab >= 0 && hidden >= 0 && vocab <= 0x7fffffff, DOE_E_INVALID,
                "bad gather shape");
    const long total = (long)n_ids * hidden;
    if (total == 0) return DOE_OK;
    DOE_REQUIRE(table_f16 && ids && output, DOE_E_INVALID, "null pointer");
    hipLaunchKernelGGL(embed_kernel, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream,
                       (const _Float16 *)table_f16, ids, output, (int)n_ids, (int)vocab, (int)hidden,
                       scale);
    DOE_LAUNCH_CHECK("embed_kernel");
    return DOE_OK;
}

}  // extern "C"
