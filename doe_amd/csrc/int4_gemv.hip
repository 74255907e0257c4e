// int4_gemv.hip -- symmetric int4 group-32 GEMV for batch decode (M <= 8) on gfx950.
//
// y[b][n] = sum_k (q[n][k] - 8) * s[n][k/32] * x[b][k]: q packed eight nibbles
// per u32, element k of row n at bits 4*(k%8) of word (n*K + k)/8, f16 scales
// [n][K/32], x f32 [M][K], y f32 [M][N] -- complex_fused_gemv_dequant.wgsl:18-23
// (nibble - 8) and :25-66 (GEMV over the row, scale [row][col/group]), with the
// f16 scales of the 27B-class batch-8 decode shape.
//
// One v_mfma_f32_16x16x32_f16 per (16 rows, one 32-element group):
//   * A = the x image: 16 columns = the eight batch rows' x_hi and x_lo (x
//     scaled per batch row by a power of two so its max sits near 2^14, split
//     into two f16), in the k order of B below;
//   * B = the nibbles of one u32 per lane as f16 subnormals with ANDs only:
//     w & 0x000F000F holds nibbles 0 and 4 as q * 2^-24, w & 0x00F000F0 nibbles
//     1 and 5 as q * 2^-20 (the image holds x / 16 there, exact), and the same
//     of w >> 8 nibbles 2, 6 and 3, 7: every product is exact;
//   * D + C, C = -8 * 2^-24 * sum(x) of the group in the x_hi columns, is
//     2^-24 * sum((q - 8) x).
// D lands with lane (row, column group) holding four batch columns of one
// row: one f16 scale (v_fma_mix) serves all four.  The power-of-two unscale
// per batch row and the hi + lo sum (one cross-half lane swap) come at the
// end.
//
// A pre-pass (one workgroup per batch row and 64 groups) finds the row's max |x| and writes
// the image ([group][64 lanes][8 f16], 1 KB per group), the corrections
// ([group][16] f32) and the row's scale exponent.  A workgroup of the GEMV
// owns 64 rows (four 16-row tiles per wave, so an image fragment feeds four
// MFMAs) and 32 groups of K, eight per wave with every load of a wave issued
// up front; the four waves' sums meet in LDS.  K is split over the grid's y
// dimension into 32-group ranges whose sums are added atomically into y (the
// pre-pass clears it), so the f32 summation order varies from run to run.
#include "common.h"

#include <math.h>
#include <mutex>

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxBatch = 8;

// Pre-pass: workgroup (b, p) = batch row b (rows >= M write zeros), groups
// [64 p, 64 p + 64); every part of a row finds the row's maximum itself (the
// same exact value, so the same exponent).  When the GEMV splits K (atomic
// partial sums), the parts also clear y[b].
constexpr int kImgThreads = 256;
constexpr int kImgGroups = 64;  // groups per workgroup: one item per thread
__global__ __launch_bounds__(kImgThreads) void int4_x_image_kernel(const float *__restrict__ x,
                                                                   _Float16 *__restrict__ img,
                                                                   float *__restrict__ corr,
                                                                   int *__restrict__ sig_out,
                                                                   float *__restrict__ y_clear,
                                                                   int M, int N, int K) {
    __shared__ float wmax[kImgThreads / 64];
    const int b = blockIdx.x, part = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    if (y_clear && b < M) {
        const int chunk = (N + (int)gridDim.y - 1) / (int)gridDim.y, i1 = min(N, (part + 1) * chunk);
        for (int i = part * chunk + tid; i < i1; i += kImgThreads) y_clear[(size_t)b * N + i] = 0.0f;
    }
    const int G = K / 32;
    const int g0 = part * kImgGroups, g1 = min(G, g0 + kImgGroups);
    const bool live = b < M;
    const float *xr = x + (size_t)(live ? b : 0) * K;
    float amax = 0.0f;
    if (live)
#pragma unroll 8
        for (int k4 = tid; k4 < K / 4; k4 += kImgThreads) {  // eight loads in flight per thread
            const float4 v = reinterpret_cast<const float4 *>(xr)[k4];
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    if (lane == 0) wmax[tid >> 6] = amax;
    __syncthreads();
    amax = 0.0f;
#pragma unroll
    for (int i = 0; i < kImgThreads / 64; ++i) amax = fmaxf(amax, wmax[i]);
    int sig = 0;
    if (amax > 0.0f && amax <= 3.0e38f) {
        sig = 14 - __builtin_amdgcn_frexp_expf(amax);
        sig = sig < -120 ? -120 : (sig > 120 ? 120 : sig);
    }
    if (tid == 0 && part == 0) sig_out[b] = sig;
    const float sc = __builtin_amdgcn_ldexpf(1.0f, sig);
    // item (g, kg): eight consecutive x, four items per group in one quad
    for (int item = g0 * 4 + tid; item < g1 * 4; item += kImgThreads) {
        const int g = item >> 2, kg = item & 3;
        float v[8];
        if (live) {
            const float4 p0 = reinterpret_cast<const float4 *>(xr + 32 * g + 8 * kg)[0];
            const float4 p1 = reinterpret_cast<const float4 *>(xr + 32 * g + 8 * kg)[1];
            v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w; v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = 0.0f;
        }
        float sum = 0.0f;
        half8 hi, lo;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // slot j: nibble (j / 2) + 4 (j % 2) ... in B's order n0 n4 n1 n5 n2 n6 n3 n7
            const int nib = (j >> 1) + 4 * (j & 1);
            const float t = v[nib] * sc;
            sum += t;
            const _Float16 h = (_Float16)t, l = (_Float16)(t - (float)h);
            // slots 2, 3, 6, 7 meet nibbles coded at bits 4..7 (x 16): store x / 16
            const bool odd = (j & 2) != 0;
            hi[j] = odd ? (_Float16)((float)h * 0.0625f) : h;
            lo[j] = odd ? (_Float16)((float)l * 0.0625f) : l;
        }
        _Float16 *base = img + (size_t)g * 512;
        *reinterpret_cast<half8 *>(base + (kg * 16 + b) * 8) = hi;
        *reinterpret_cast<half8 *>(base + (kg * 16 + 8 + b) * 8) = lo;
        // the group's sum over its four quads (consecutive threads)
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        if (kg == 0) {
            corr[g * 16 + b] = -8.0f * 5.9604644775390625e-08f * sum;  // -8 * 2^-24 * sum(x)
            corr[g * 16 + 8 + b] = 0.0f;
        }
    }
}

// B operand of one word: halves (n0, n4, 16 n1, 16 n5, n2, n6, 16 n3, 16 n7) * 2^-24.
__device__ __forceinline__ half8 unpack_int4(uint32_t w) {
    const uint32_t w8 = w >> 8;
    return __builtin_bit_cast(half8, u32x4{w & 0x000f000fu, w & 0x00f000f0u, w8 & 0x000f000fu, w8 & 0x00f000f0u});
}

struct Int4Args {
    const uint32_t *q;
    const uint16_t *scales;
    const _Float16 *img;
    const float *corr;
    const int *sig;
    float *out;  // y [M][N] (K splits add atomically into y, cleared by the pre-pass)
    int M, N, K, G;
};

// 64 rows x (4 GPW) groups per workgroup; wave w takes groups
// [blockIdx.y 4 GPW + w GPW, + GPW).  A row's GPW groups are GPW * 16
// contiguous bytes: the wave reads them with whole-line 16-byte loads (GPW
// lanes per row) and regroups them through its own LDS slice into the MFMA
// lane order (lane (r, j) takes word j of each group of row r).
template <int GPW>
__global__ __launch_bounds__(256) void int4_gemv_kernel(Int4Args a) {
    static_assert(GPW == 8, "one 16-byte scale load per row tile covers eight groups");
    __shared__ float red[3][4][4][64];
    __shared__ __attribute__((aligned(16))) uint32_t wl[4][64 * 4 * GPW];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int r0 = blockIdx.x * 64;
    const int g0 = (blockIdx.y * 4 + wave) * GPW;
    const bool active = g0 < a.G;  // a.G is a multiple of GPW
    const int gb = active ? g0 : 0;

    // all loads first: the x image fragments and corrections (L2-resident),
    // the scales of this lane's rows, then the 64 rows' weight bytes
    half8 xa[GPW];
    float4v cz[GPW];
#pragma unroll
    for (int u = 0; u < GPW; ++u) {
        xa[u] = *reinterpret_cast<const half8 *>(a.img + ((size_t)(gb + u) * 64 + lane) * 8);
        cz[u] = *reinterpret_cast<const float4v *>(a.corr + (gb + u) * 16 + 4 * lg);
    }
    u32x4 sv[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
        sv[t] = *reinterpret_cast<const u32x4 *>(a.scales + (size_t)min(r0 + 16 * t + lr, a.N - 1) * a.G + gb);
    constexpr int RPI = 64 / GPW;  // rows per load instruction
    u32x4 wg[GPW];
#pragma unroll
    for (int j = 0; j < GPW; ++j) {
        const int row = j * RPI + lane / GPW;
        wg[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(
            a.q + (size_t)min(r0 + row, a.N - 1) * (a.K / 8) + 4 * (gb + lane % GPW)));
    }
    // regroup: wl[(row * 4 + word) * GPW + group]
    uint32_t *my = wl[wave];
#pragma unroll
    for (int j = 0; j < GPW; ++j) {
        const int row = j * RPI + lane / GPW, u = lane % GPW;
#pragma unroll
        for (int e = 0; e < 4; ++e) my[(row * 4 + e) * GPW + u] = wg[j][e];
    }
    // (each wave reads back only its own slice: no workgroup barrier needed)
    uint32_t w[4][GPW];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const u32x4 *src = reinterpret_cast<const u32x4 *>(my + ((16 * t + lr) * 4 + lg) * GPW);
#pragma unroll
        for (int h = 0; h < GPW / 4; ++h) {
            const u32x4 v = src[h];
            w[t][4 * h] = v.x;
            w[t][4 * h + 1] = v.y;
            w[t][4 * h + 2] = v.z;
            w[t][4 * h + 3] = v.w;
        }
    }

    // acc[t][i]: row r0 + 16 t + lr, column 4 lg + i (batch (4 lg + i) % 8, hi for lg < 2)
    float acc[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] = 0.0f;
    if (active) {
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                // (the correction is added after the product: as the MFMA's
                // accumulator input it cost precision, rel-L2 1.9e-5 vs 4.8e-6)
                const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
                const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[u], unpack_int4(w[t][u]), zero, 0, 0, 0) + cz[u];
                const uint32_t pair = sv[t][u >> 1];
                const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)((u & 1) ? (pair >> 16) : pair));
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(s, d[i], acc[t][i]);
            }
        }
    }
    // the four waves' partial sums meet in wave 0
    if (wave > 0) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave - 1][t][i][lane] = acc[t][i];
    }
    __syncthreads();
    if (wave > 0) return;
    // x_hi columns sit in lanes 0..31, x_lo in 32..63: one swap adds them
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = acc[t][i] + red[0][t][i][lane] + red[1][t][i][lane] + red[2][t][i][lane];
            auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            v = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
            const int b = 4 * lg + i, row = r0 + 16 * t + lr;
            if (lg < 2 && b < a.M && row < a.N) {
                const float r = __builtin_amdgcn_ldexpf(v, 24 - a.sig[b]);
                if (gridDim.y > 1) atomicAdd(a.out + (size_t)b * a.N + row, r);  // y cleared by the pre-pass
                else a.out[(size_t)b * a.N + row] = r;
            }
        }
}

// Lane (row, q) holds the four words of group g + q of its row (one 16-byte
// load); returns in out[i] word q of group g + i -- group g + i's B operand
// (lane (row, w) must hold word w).  A 4 x 4 transpose across the lane
// quarters: one 32-lane and one 16-lane swap stage.
__device__ __forceinline__ void quad_transpose(const u32x4 v, uint32_t out[4]) {
    const auto s02 = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
    const auto s13 = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
    const auto t01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
    const auto t23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
    out[0] = t01[0];
    out[1] = t01[1];
    out[2] = t23[0];
    out[3] = t23[1];
}

// Streaming form: a workgroup owns one K range of 4 GPW groups (wave w the
// GPW groups from 4 GPW split + w GPW) and walks the row blocks
// j, j + wps, j + 2 wps, ... of 64 rows.  The wave's x image fragments and
// corrections are loaded once; each row block's weights and scales are loaded
// while the previous block is computed (two register sets), straight into the
// MFMA layout: lane (row, q) loads the 16 bytes of group 4h + q of its row
// and a lane-quarter transpose hands every lane its word of each group.  The
// four waves' sums meet in LDS (double-buffered, one barrier per block), each
// wave summing and adding one 16-row tile into y.
template <int GPW>
__global__ __launch_bounds__(256, 2) void int4_gemv_stream_kernel(Int4Args a, int wps, int row_blocks) {
    static_assert(GPW == 8, "one 16-byte scale load per row tile covers eight groups");
    __shared__ float red[2][4][4][4][64];  // [buffer][source wave][tile][column][lane]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int sp = blockIdx.x / wps, j = blockIdx.x - sp * wps;
    const int g0 = (sp * 4 + wave) * GPW;
    const bool active = g0 < a.G;  // a.G is a multiple of GPW
    const int gb = active ? g0 : 0;

    half8 xa[GPW];
    float4v cz[GPW];
#pragma unroll
    for (int u = 0; u < GPW; ++u) {
        xa[u] = *reinterpret_cast<const half8 *>(a.img + ((size_t)(gb + u) * 64 + lane) * 8);
        cz[u] = *reinterpret_cast<const float4v *>(a.corr + (gb + u) * 16 + 4 * lg);
    }
    const size_t row_words = (size_t)a.K / 8;
    u32x4 wq[2][4][GPW / 4], sv[2][4];
    auto load = [&](const int set, const int rb) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int row = min(rb * 64 + 16 * t + lr, a.N - 1);
            sv[set][t] = *reinterpret_cast<const u32x4 *>(a.scales + (size_t)row * a.G + gb);
#pragma unroll
            for (int h = 0; h < GPW / 4; ++h)
                wq[set][t][h] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4 *>(a.q + row * row_words + 4 * (gb + 4 * h + lg)));
        }
    };
    auto step = [&](const int cur, const int rb) __attribute__((always_inline)) {
        if (rb + wps < row_blocks) load(cur ^ 1, rb + wps);
        // acc[t][i]: row 64 rb + 16 t + lr, column 4 lg + i (batch (4 lg + i) % 8, hi for lg < 2)
        float acc[4][4];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][i] = 0.0f;
        if (active) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int h = 0; h < GPW / 4; ++h) {
                    uint32_t wv[4];
                    quad_transpose(wq[cur][t][h], wv);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int u = 4 * h + q;
                        // (the correction is added after the product: as the MFMA's
                        // accumulator input it cost precision, rel-L2 1.9e-5 vs 4.8e-6)
                        const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
                        const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[u], unpack_int4(wv[q]), zero, 0, 0, 0) + cz[u];
                        const uint32_t pair = sv[cur][t][u >> 1];
                        const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)((u & 1) ? (pair >> 16) : pair));
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(s, d[i], acc[t][i]);
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[cur][wave][t][i][lane] = acc[t][i];
        __syncthreads();
        // wave w sums row tile w over the four waves; x_hi columns sit in lanes
        // 0..31, x_lo in 32..63: one swap adds them
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = (red[cur][0][wave][i][lane] + red[cur][1][wave][i][lane]) +
                      (red[cur][2][wave][i][lane] + red[cur][3][wave][i][lane]);
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            v = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
            const int b = 4 * lg + i, row = rb * 64 + 16 * wave + lr;
            if (lg < 2 && b < a.M && row < a.N) {
                const float r = __builtin_amdgcn_ldexpf(v, 24 - a.sig[b]);
                if (a.G > 4 * GPW) atomicAdd(a.out + (size_t)b * a.N + row, r);  // y cleared by the pre-pass
                else a.out[(size_t)b * a.N + row] = r;
            }
        }
    };
    int rb = j;
    if (rb >= row_blocks) return;
    load(0, rb);
    for (;;) {
        step(0, rb);
        rb += wps;
        if (rb >= row_blocks) break;
        step(1, rb);
        rb += wps;
        if (rb >= row_blocks) break;
    }
}

std::mutex g_ws_mu;
void *g_ws = nullptr;
size_t g_ws_bytes = 0;
int g_num_cus = 0;
int g_int4_kernel = 0;  // 0 automatic, 1 one-shot workgroups, 2 streaming

}  // namespace

extern "C" {

int doe_int4g32_gemv(const uint32_t *w_u4, const uint16_t *scales_f16, const float *x, float *y,
                     int64_t m, int64_t n, int64_t k, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(m >= 1 && m <= kMaxBatch, DOE_E_UNSUPPORTED, "int4g32_gemv supports batch 1..8 (got %lld)",
                (long long)m);
    DOE_REQUIRE(n >= 0 && k >= 0, DOE_E_INVALID, "negative shape");
    if (n == 0) return DOE_OK;
    DOE_REQUIRE(y, DOE_E_INVALID, "null output");
    hipStream_t st = (hipStream_t)stream;
    if (k == 0) {
        return doe::fill_bytes_async(y, 0, (size_t)m * n * sizeof(float), st);
    }
    DOE_REQUIRE(w_u4 && scales_f16 && x, DOE_E_INVALID, "null pointer");
    DOE_REQUIRE(k % 256 == 0, DOE_E_UNSUPPORTED, "int4g32_gemv needs k %% 256 == 0 (got %lld)", (long long)k);
    DOE_REQUIRE(n <= (1 << 26) && k <= (1 << 24), DOE_E_UNSUPPORTED, "int4g32_gemv shape too large");
    DOE_REQUIRE((((uintptr_t)w_u4 | (uintptr_t)scales_f16 | (uintptr_t)x) & 15) == 0, DOE_E_INVALID,
                "weights, scales and x must be 16-byte aligned");
    if (g_num_cus == 0) {
        int dev = 0, cus = 0;
        DOE_HIP_CHECK(hipGetDevice(&dev));
        DOE_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        g_num_cus = cus > 0 ? cus : 256;
    }
    const int G = (int)(k / 32);
    const int row_blocks = (int)((n + 63) / 64);
    // eight groups per wave (every load of a wave in flight at once), K split
    // over the grid so that the rows times the splits fill the CUs
    const int gpw = 8;
    const int per_wg = 4 * gpw;
    const int splits = (G + per_wg - 1) / per_wg;

    const size_t img_bytes = (size_t)G * 64 * 8 * 2;
    const size_t fac_bytes = (size_t)G * 16 * 4 + kMaxBatch * 4;  // corrections, exponents
    const size_t need = img_bytes + fac_bytes;
    void *ws;
    {
        std::lock_guard<std::mutex> lk(g_ws_mu);
        if (g_ws_bytes < need) {
            if (g_ws) {
                // queued kernels (any stream) may still read the old workspace
                DOE_HIP_CHECK(hipDeviceSynchronize());
                DOE_HIP_CHECK(hipFree(g_ws));
            }
            g_ws = nullptr;
            g_ws_bytes = 0;
            DOE_HIP_CHECK(hipMalloc(&g_ws, need));
            g_ws_bytes = need;
        }
        ws = g_ws;
    }
    _Float16 *img = (_Float16 *)ws;
    float *corr = (float *)((char *)ws + img_bytes);
    int *sig = (int *)(corr + (size_t)G * 16);
    const int img_parts = G > 0 ? (G + kImgGroups - 1) / kImgGroups : 1;
    hipLaunchKernelGGL(int4_x_image_kernel, dim3(kMaxBatch, (unsigned)img_parts), dim3(kImgThreads), 0, st, x, img, corr, sig,
                       splits > 1 ? y : nullptr, (int)m, (int)n, (int)k);
    DOE_LAUNCH_CHECK("int4_x_image_kernel");
    Int4Args a;
    a.q = w_u4;
    a.scales = scales_f16;
    a.img = img;
    a.corr = corr;
    a.sig = sig;
    a.out = y;
    a.M = (int)m;
    a.N = (int)n;
    a.K = (int)k;
    a.G = G;
    // the streaming form pays off once every workgroup walks several row blocks
    // (measured at batch 8: 25600 x 5120 and 5120 x 25600 faster, 9216 x 5120
    // slower than the one-shot form)
    const int64_t items = (int64_t)row_blocks * splits;
    const bool stream_ok = items >= 6 * (int64_t)g_num_cus;
    if (g_int4_kernel == 1 || (g_int4_kernel == 0 && !stream_ok)) {
        const dim3 grid((unsigned)row_blocks, (unsigned)splits);
        hipLaunchKernelGGL(int4_gemv_kernel<8>, grid, dim3(256), 0, st, a);
    } else {
        // about two workgroups per CU, each K range's row blocks dealt evenly
        const int64_t per_wg = (items + 2 * g_num_cus - 1) / (2 * g_num_cus);
        const int wps = (int)((row_blocks + per_wg - 1) / per_wg);
        hipLaunchKernelGGL(int4_gemv_stream_kernel<8>, dim3((unsigned)(wps * splits)), dim3(256), 0, st, a, wps,
                           row_blocks);
    }
    DOE_LAUNCH_CHECK("int4_gemv_kernel");
    return DOE_OK;
}

}  // extern "C"

namespace doe {

int int4_set_kernel(int v) {
    DOE_REQUIRE(v >= 0 && v <= 2, DOE_E_INVALID, "int4_gemv.kernel is 0, 1 or 2");
    g_int4_kernel = v;
    return DOE_OK;
}

}  // namespace doe
