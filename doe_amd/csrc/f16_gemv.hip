// f16_gemv.hip -- f16-weight GEMV (the lm_head) for gfx950.
//
// C[n] = alpha * sum_k A[k] * f32(B[n*K + k]) with B f16 [N][K] row-major
// (runtime/zig/tests/tsir/real/lm_head_gemv/lm_head_gemv.wgsl:78-180,
// transpose_b = 1), A and C f32.
//
// doe_lm_head_gemv is the full form: m activation rows, either layout of B
// (transpose_b), any k; one row against [N][K] takes the kernel below.
//
// Decomposition: persistent waves; a wave owns whole rows (row = wave id +
// i * total waves) and each lane a fixed set of 16-byte pieces of the row
// (pieces lane, lane + 64, ...), so its 8-element activation slices stay in
// VGPRs for the whole kernel, split into f16 hi/lo pairs (~22 significant
// bits).  A row is U 16-byte loads per lane, v_dot2c_f32_f16 against the hi
// and lo pairs, and one wave reduction.  Two rows are processed per step and
// the next step's rows are loaded before the current ones are reduced.
#include "common.h"

#include <math.h>

namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, a), __builtin_bit_cast(half2v, b), c,
                                  false);
}

__device__ __forceinline__ uint32_t pack2(_Float16 lo, _Float16 hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

__device__ __forceinline__ u32x4 load16(const uint16_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

template <int P>
__device__ __forceinline__ float row_dot(const u32x4 (&w)[P], const uint32_t (&xh)[P][4],
                                         const uint32_t (&xl)[P][4]) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < P; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a0 = dot2(w[i][j], xh[i][j], a0);
            a1 = dot2(w[i][j], xl[i][j], a1);
        }
    }
    return a0 + a1;
}

// Argmax keys (see elementwise.hip): ordered float bits high, inverted index
// low; the unsigned max is the largest logit at the lowest index; NaN never wins.
__device__ __forceinline__ unsigned long long argmax_key(float v, unsigned idx) {
    if (v != v) return 0ull;
    unsigned u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (0xffffffffu - idx);
}

// Optional fusions: RMSNorm of the activation (every wave holds the whole
// activation, so it normalises on its own) and a per-workgroup argmax
// partial (the greedy sample over the output).
struct F16Fusion {
    const float *norm_w;
    float norm_eps;
    int norm_offset;
    unsigned long long *argmax_part;  // [gridDim.x] best key per workgroup
};

template <int P>
__global__ __launch_bounds__(256) void f16_gemv_kernel(const uint16_t *__restrict__ b,
                                                       const float *__restrict__ a,
                                                       float *__restrict__ c, int n, int k,
                                                       float alpha, F16Fusion fz) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nwaves = gridDim.x * 4;
    const int npieces = k >> 3;

    // activation slices of this lane; pieces past k are zero
    float xs[P][8];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int p = lane + 64 * i;
        const bool ok = p < npieces;
        const float4 *src = reinterpret_cast<const float4 *>(a + 8 * (ok ? p : 0));
        const float4 lo4 = src[0], hi4 = src[1];
        const float v[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) xs[i][j] = ok ? v[j] : 0.0f;
    }
    if (fz.norm_w) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < P; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) ss = fmaf(xs[i][j], xs[i][j], ss);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        const float inv = 1.0f / sqrtf(ss / (float)k + fz.norm_eps);
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int p = min(lane + 64 * i, npieces - 1);
            const float4 *ws = reinterpret_cast<const float4 *>(fz.norm_w + 8 * p);
            const float4 w0 = ws[0], w1 = ws[1];
            const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) xs[i][j] = xs[i][j] * inv * (fz.norm_offset ? 1.0f + wv[j] : wv[j]);
        }
    }

    // f16 hi/lo pairs
    uint32_t xh[P][4], xl[P][4];
#pragma unroll
    for (int i = 0; i < P; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float x0 = xs[i][2 * j], x1 = xs[i][2 * j + 1];
            const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
            xh[i][j] = pack2(h0, h1);
            xl[i][j] = pack2((_Float16)(x0 - (float)h0), (_Float16)(x1 - (float)h1));
        }
    }

    // rows of this wave: wave, wave + nwaves, ...; two per step, prefetched
    u32x4 w0[P], w1[P];
    int row = wave;
    auto load_rows = [&](int r, u32x4 (&d0)[P], u32x4 (&d1)[P]) {
        const int r0 = min(r, n - 1), r1 = min(r + nwaves, n - 1);
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int p = min(lane + 64 * i, npieces - 1);
            d0[i] = load16(b + (size_t)r0 * k + 8 * p);
            d1[i] = load16(b + (size_t)r1 * k + 8 * p);
        }
    };
    unsigned long long best = 0;
    if (row < n) load_rows(row, w0, w1);
    for (; row < n; row += 2 * nwaves) {
        u32x4 n0[P], n1[P];
        load_rows(row + 2 * nwaves, n0, n1);
        // pieces past k were clamped onto a valid piece: mask them out
#pragma unroll
        for (int i = 0; i < P; ++i) {
            if (lane + 64 * i >= npieces) {
                w0[i] = u32x4{0, 0, 0, 0};
                w1[i] = u32x4{0, 0, 0, 0};
            }
        }
        float s0 = row_dot<P>(w0, xh, xl);
        float s1 = row_dot<P>(w1, xh, xl);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            s0 += __shfl_xor(s0, o, 64);
            s1 += __shfl_xor(s1, o, 64);
        }
        s0 *= alpha;
        s1 *= alpha;
        if (lane == 0 && c) {
            c[row] = s0;
            if (row + nwaves < n) c[row + nwaves] = s1;
        }
        best = argmax_key(s0, (unsigned)row) > best ? argmax_key(s0, (unsigned)row) : best;
        if (row + nwaves < n) {
            const unsigned long long k1 = argmax_key(s1, (unsigned)(row + nwaves));
            best = k1 > best ? k1 : best;
        }
#pragma unroll
        for (int i = 0; i < P; ++i) {
            w0[i] = n0[i];
            w1[i] = n1[i];
        }
    }
    if (fz.argmax_part) {
        __shared__ unsigned long long wb[4];
        if (lane == 0) wb[threadIdx.x >> 6] = best;  // identical in every lane of the wave
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long m = wb[0];
            for (int i = 1; i < 4; ++i) m = wb[i] > m ? wb[i] : m;
            fz.argmax_part[blockIdx.x] = m;
        }
    }
}

// ---- general forms: any k, B in either layout, m activation rows -----------
//
// c[r][j] = alpha * sum_k a[r][k] * B(j, k) for r < m, with B(j, k) =
// b[j*K + k] (transpose_b = 1) or b[k*N + j] (transpose_b = 0).  Products
// are plain f32 FMAs of the exact f16 -> f32 weight; each launch covers MT
// activation rows, so the weights are read ceil(m / MT) times.

template <int VEC>
__device__ __forceinline__ void load_f16(const uint16_t *p, float (&v)[VEC]) {
    if constexpr (VEC == 8) {
        const u32x4 w = load16(p);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // copy the element out first: a bit_cast of the element
            // expression itself reads element 0 of w
            const uint32_t word = w[j];
            const half2v h = __builtin_bit_cast(half2v, word);
            v[2 * j] = (float)h[0];
            v[2 * j + 1] = (float)h[1];
        }
    } else {
        v[0] = (float)__builtin_bit_cast(_Float16, *p);
    }
}

// transpose_b = 0, b [K][N]: a lane owns VEC adjacent columns, the four
// waves of a workgroup take the k rows w, w + 4, ... (each row a contiguous
// 64 * VEC * 2-byte run) and fold their partial sums through LDS.
template <int MT, int VEC>
__global__ __launch_bounds__(256) void lm_head_kn_kernel(const float *__restrict__ a,
                                                         const uint16_t *__restrict__ b,
                                                         float *__restrict__ c, int m, int n,
                                                         int k, float alpha) {
    __shared__ float red[3][MT * VEC][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = (blockIdx.x * 64 + lane) * VEC;
    const int row0 = blockIdx.y * MT;
    const bool live = col < n;
    const uint16_t *bc = b + (live ? col : 0);
    float acc[MT][VEC];
#pragma unroll
    for (int r = 0; r < MT; ++r)
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[r][v] = 0.0f;
    int kk = wave;
    for (; kk + 12 < k; kk += 16) {
        float w[4][VEC];
#pragma unroll
        for (int u = 0; u < 4; ++u) load_f16<VEC>(bc + (size_t)(kk + 4 * u) * n, w[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int r = 0; r < MT; ++r) {
                const float x = row0 + r < m ? a[(size_t)(row0 + r) * k + kk + 4 * u] : 0.0f;
#pragma unroll
                for (int v = 0; v < VEC; ++v) acc[r][v] = fmaf(x, w[u][v], acc[r][v]);
            }
    }
    for (; kk < k; kk += 4) {
        float w[VEC];
        load_f16<VEC>(bc + (size_t)kk * n, w);
#pragma unroll
        for (int r = 0; r < MT; ++r) {
            const float x = row0 + r < m ? a[(size_t)(row0 + r) * k + kk] : 0.0f;
#pragma unroll
            for (int v = 0; v < VEC; ++v) acc[r][v] = fmaf(x, w[v], acc[r][v]);
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < MT; ++r)
#pragma unroll
            for (int v = 0; v < VEC; ++v) red[wave - 1][r * VEC + v][lane] = acc[r][v];
    }
    __syncthreads();
    if (wave == 0 && live) {
#pragma unroll
        for (int r = 0; r < MT; ++r) {
            if (row0 + r >= m) break;
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
                const float s = ((acc[r][v] + red[0][r * VEC + v][lane]) + red[1][r * VEC + v][lane]) +
                                red[2][r * VEC + v][lane];
                c[(size_t)(row0 + r) * n + col + v] = s * alpha;
            }
        }
    }
}

// transpose_b = 1, b [N][K], any k: a wave owns two rows of b at a time and
// its lanes stride along k, VEC elements per lane per step.
template <int MT, int VEC>
__global__ __launch_bounds__(256) void lm_head_nk_kernel(const float *__restrict__ a,
                                                         const uint16_t *__restrict__ b,
                                                         float *__restrict__ c, int m, int n,
                                                         int k, float alpha) {
    const int lane = threadIdx.x & 63;
    const int j0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 2;
    if (j0 >= n) return;
    const int j1 = min(j0 + 1, n - 1);
    const int row0 = blockIdx.y * MT;
    const uint16_t *b0 = b + (size_t)j0 * k, *b1 = b + (size_t)j1 * k;
    float acc[MT][2];
#pragma unroll
    for (int r = 0; r < MT; ++r) acc[r][0] = acc[r][1] = 0.0f;
    for (int kk = lane * VEC; kk < k; kk += 64 * VEC) {
        float w0[VEC], w1[VEC];
        load_f16<VEC>(b0 + kk, w0);
        load_f16<VEC>(b1 + kk, w1);
#pragma unroll
        for (int r = 0; r < MT; ++r) {
            if (row0 + r >= m) break;
            const float *ar = a + (size_t)(row0 + r) * k + kk;
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
                acc[r][0] = fmaf(ar[v], w0[v], acc[r][0]);
                acc[r][1] = fmaf(ar[v], w1[v], acc[r][1]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < MT; ++r) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            acc[r][0] += __shfl_xor(acc[r][0], o, 64);
            acc[r][1] += __shfl_xor(acc[r][1], o, 64);
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < MT; ++r) {
            if (row0 + r >= m) break;
            c[(size_t)(row0 + r) * n + j0] = acc[r][0] * alpha;
            if (j0 + 1 < n) c[(size_t)(row0 + r) * n + j0 + 1] = acc[r][1] * alpha;
        }
    }
}

template <int MT>
int lm_head_general(const float *a, const uint16_t *b, float *c, int m, int n, int k, float alpha,
                    int transpose_b, hipStream_t st) {
    const unsigned mtiles = (unsigned)((m + MT - 1) / MT);
    if (transpose_b) {
        const bool v8 = (k % 8) == 0 && ((uintptr_t)b & 15) == 0;
        const dim3 grid((unsigned)((n + 7) / 8), mtiles), blk(256);
        if (v8)
            hipLaunchKernelGGL((lm_head_nk_kernel<MT, 8>), grid, blk, 0, st, a, b, c, m, n, k, alpha);
        else
            hipLaunchKernelGGL((lm_head_nk_kernel<MT, 1>), grid, blk, 0, st, a, b, c, m, n, k, alpha);
        DOE_LAUNCH_CHECK("lm_head_nk_kernel");
    } else {
        const bool v8 = (n % 8) == 0 && ((uintptr_t)b & 15) == 0;
        const int cols = v8 ? 512 : 64;
        const dim3 grid((unsigned)((n + cols - 1) / cols), mtiles), blk(256);
        if (v8)
            hipLaunchKernelGGL((lm_head_kn_kernel<MT, 8>), grid, blk, 0, st, a, b, c, m, n, k, alpha);
        else
            hipLaunchKernelGGL((lm_head_kn_kernel<MT, 1>), grid, blk, 0, st, a, b, c, m, n, k, alpha);
        DOE_LAUNCH_CHECK("lm_head_kn_kernel");
    }
    return DOE_OK;
}

int g_num_cus = 0;

int f16_launch(const uint16_t *b_f16, const float *a, float *c, int64_t n, int64_t k, float alpha,
               const F16Fusion &fz, hipStream_t st, long max_blocks, unsigned *blocks_out) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(n >= 0 && k >= 0 && n <= 0x7fffffff, DOE_E_INVALID, "bad f16_gemv shape");
    if (n == 0) return DOE_OK;
    DOE_REQUIRE(c || fz.argmax_part, DOE_E_INVALID, "null output");
    if (k == 0) {
        DOE_REQUIRE(c && !fz.argmax_part, DOE_E_UNSUPPORTED, "k == 0 with argmax");
        return doe::fill_bytes_async(c, 0, (size_t)n * 4, st);
    }
    DOE_REQUIRE(b_f16 && a, DOE_E_INVALID, "null pointer");
    DOE_REQUIRE((k % 8) == 0 && k <= 64 * 8 * 16, DOE_E_UNSUPPORTED,
                "f16_gemv needs k %% 8 == 0 and k <= 8192 (got %lld)", (long long)k);
    DOE_REQUIRE(((uintptr_t)b_f16 & 15) == 0 && ((uintptr_t)a & 15) == 0 &&
                    ((uintptr_t)fz.norm_w & 15) == 0,
                DOE_E_INVALID, "weights, activation and norm weight must be 16-byte aligned");
    if (g_num_cus == 0) {
        int dev = 0, cus = 0;
        DOE_HIP_CHECK(hipGetDevice(&dev));
        DOE_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        g_num_cus = cus > 0 ? cus : 256;
    }
    const int pieces = (int)(k / 8);
    const int p = (pieces + 63) / 64;
    long waves = (n + 1) / 2;
    long blocks = (waves + 3) / 4;
    const long cap = (long)g_num_cus * 4;  // persistent: 16 waves per CU
    if (blocks > cap) blocks = cap;
    if (max_blocks > 0 && blocks > max_blocks) blocks = max_blocks;
    if (blocks_out) *blocks_out = (unsigned)blocks;
    const dim3 grid((unsigned)blocks), blk(256);
    switch (p) {
#define DOE_F16_CASE(PP) \
    case PP: hipLaunchKernelGGL(f16_gemv_kernel<PP>, grid, blk, 0, st, b_f16, a, c, (int)n, (int)k, alpha, fz); break;
        DOE_F16_CASE(1) DOE_F16_CASE(2) DOE_F16_CASE(3) DOE_F16_CASE(4) DOE_F16_CASE(5)
        DOE_F16_CASE(6) DOE_F16_CASE(7) DOE_F16_CASE(8) DOE_F16_CASE(9) DOE_F16_CASE(10)
        DOE_F16_CASE(11) DOE_F16_CASE(12) DOE_F16_CASE(13) DOE_F16_CASE(14) DOE_F16_CASE(15)
        DOE_F16_CASE(16)
#undef DOE_F16_CASE
        default: return doe::set_error(DOE_E_UNSUPPORTED, "k too large");
    }
    DOE_LAUNCH_CHECK("f16_gemv_kernel");
    return DOE_OK;
}

}  // namespace

extern "C" {

int doe_f16_gemv(const uint16_t *b_f16, const float *a, float *c, int64_t n, int64_t k, float alpha,
                 doe_stream_t stream) {
    const F16Fusion fz{nullptr, 0.0f, 0, nullptr};
    return f16_launch(b_f16, a, c, n, k, alpha, fz, (hipStream_t)stream, 0, nullptr);
}

int doe_f16_gemv_argmax(const uint16_t *b_f16, const float *a, float *logits, int64_t n, int64_t k,
                        float alpha, const float *norm_weight, float norm_eps, int norm_weight_offset,
                        uint64_t *argmax_partials, int64_t partials_capacity, int32_t *num_partials,
                        doe_stream_t stream) {
    DOE_REQUIRE(argmax_partials && partials_capacity >= 1024, DOE_E_INVALID,
                "argmax partials need room for 1024 keys");
    const F16Fusion fz{norm_weight, norm_eps, norm_weight_offset, (unsigned long long *)argmax_partials};
    unsigned blocks = 0;
    const long cap = partials_capacity > 0x7fffffff ? 0x7fffffffL : (long)partials_capacity;
    int rc = f16_launch(b_f16, a, logits, n, k, alpha, fz, (hipStream_t)stream, cap, &blocks);
    if (num_partials) *num_partials = (int32_t)blocks;
    return rc;
}

int doe_lm_head_gemv(const float *a, const uint16_t *b_f16, float *c, int64_t m, int64_t n,
                     int64_t k, float alpha, int transpose_b, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(m >= 0 && n >= 0 && k >= 0 && n <= 0x7fffffff && k <= (1L << 30), DOE_E_INVALID,
                "bad lm_head_gemv shape");
    DOE_REQUIRE(transpose_b == 0 || transpose_b == 1, DOE_E_INVALID, "transpose_b must be 0 or 1");
    DOE_REQUIRE(m <= 65535L * 8, DOE_E_UNSUPPORTED, "lm_head_gemv takes at most 524280 rows");
    DOE_REQUIRE((uint64_t)m * (uint64_t)n < (1ull << 40), DOE_E_INVALID, "output too large");
    hipStream_t st = (hipStream_t)stream;
    if (m == 0 || n == 0) return DOE_OK;
    DOE_REQUIRE(c, DOE_E_INVALID, "null output");
    if (k == 0) return doe::fill_bytes_async(c, 0, (size_t)m * (size_t)n * 4, st);
    DOE_REQUIRE(a && b_f16, DOE_E_INVALID, "null pointer");
    DOE_REQUIRE(((uintptr_t)a & 3) == 0 && ((uintptr_t)c & 3) == 0 && ((uintptr_t)b_f16 & 1) == 0,
                DOE_E_INVALID, "a and c must be 4-byte aligned, b 2-byte aligned");
    // one activation row against the [N][K] layout: the persistent hi/lo kernel
    if (m == 1 && transpose_b == 1 && (k % 8) == 0 && k <= 64 * 8 * 16 &&
        ((uintptr_t)b_f16 & 15) == 0 && ((uintptr_t)a & 15) == 0) {
        const F16Fusion fz{nullptr, 0.0f, 0, nullptr};
        return f16_launch(b_f16, a, c, n, k, alpha, fz, st, 0, nullptr);
    }
    if (m == 1) return lm_head_general<1>(a, b_f16, c, 1, (int)n, (int)k, alpha, transpose_b, st);
    if (m <= 4) return lm_head_general<4>(a, b_f16, c, (int)m, (int)n, (int)k, alpha, transpose_b, st);
    return lm_head_general<8>(a, b_f16, c, (int)m, (int)n, (int)k, alpha, transpose_b, st);
}

}  // extern "C"
