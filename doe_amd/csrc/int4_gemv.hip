// int4_gemv.hip -- symmetric int4 group-32 GEMV for batch decode (M <= 8) on gfx950.
//
// y[b][n] = sum_k (q[n][k] - 8) * s[n][k/32] * x[b][k]: q packed eight nibbles
// per u32, element k of row n at bits 4*(k%8) of word (n*K + k)/8, f16 scales
// [n][K/32], x f32 [M][K], y f32 [M][N] -- complex_fused_gemv_dequant.wgsl:18-23
// (nibble - 8) and :25-66 (GEMV over the row, scale [row][col/group]), with the
// f16 scales of the 27B-class batch-8 decode shape.
//
// The batch rides in the N dimension of v_mfma_f32_16x16x32_f16: one MFMA is
// 16 weight rows x one 32-element group x 16 columns, columns 0..7 carrying
// x_hi of the eight batch rows and 8..15 their x_lo (x = x_hi + x_lo in f16
// after a power-of-two scale per batch row and group), so nothing in the matrix core is
// wasted at M = 8 and the products carry ~22 bits of x.  (q - 8) is exact in
// f16 (OR the nibble into the mantissa of 1024, subtract 1032), each group's
// 16x16 result is scaled by its f16 scale in f32, and the hi/lo halves meet
// in one lane exchange at the end.
//
// A pre-pass writes x as the MFMA's B-operand image ([group][64 lanes][8 f16],
// 1 KB per group, plus one power-of-two unscale factor per group and batch
// row: x is scaled per 32-element group so max|x| sits near 2^14), read by
// every workgroup from L2.  A workgroup owns 64 rows (four 16-row MFMA tiles
// per wave, so each x fragment feeds four MFMAs) and 32 groups of K, eight
// per wave with every load of a wave issued up front; the
// four waves' sums meet in LDS.  K is split over the grid's y dimension when
// the rows alone do not fill the GPU, and the splits are summed by a small
// second kernel (deterministic order, no atomics).
#include "common.h"

#include <math.h>
#include <mutex>

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxBatch = 8;

// x image: lane l of group g holds, for column c = l % 16 (batch c % 8, part
// c / 8: 0 = hi, 1 = lo), x * 2^sig[b][g] at k = 32 g + 8 (l / 16) +
// {0, 4, 1, 5, 2, 6, 3, 7}[j]; unscale[g][c] = 2^-sig[b][g] (0 past the batch).
// One thread per (group, batch row, lane group): eight groups per workgroup.
__global__ __launch_bounds__(256) void int4_x_image_kernel(const float *__restrict__ x,
                                                           _Float16 *__restrict__ img,
                                                           float *__restrict__ unscale, int M,
                                                           int K) {
    const int lg = threadIdx.x & 3, b = (threadIdx.x >> 2) & 7;
    const int g = blockIdx.x * 8 + (threadIdx.x >> 5);
    if (g >= K / 32) return;  // whole quads leave together
    float v[8];
    if (b < M) {
        const float4 *xp = reinterpret_cast<const float4 *>(x + (size_t)b * K + 32 * g + 8 * lg);
        const float4 a = xp[0], c = xp[1];
        v[0] = a.x; v[1] = c.x; v[2] = a.y; v[3] = c.y; v[4] = a.z; v[5] = c.z; v[6] = a.w; v[7] = c.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    int sig = 0;
    if (amax > 0.0f && amax <= 3.0e38f) {
        sig = 14 - __builtin_amdgcn_frexp_expf(amax);
        sig = sig < -120 ? -120 : (sig > 120 ? 120 : sig);
    }
    const float sc = __builtin_amdgcn_ldexpf(1.0f, sig);
    _Float16 hi[8], lo[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float t = v[j] * sc;
        hi[j] = (_Float16)t;
        lo[j] = (_Float16)(t - (float)hi[j]);
    }
    _Float16 *base = img + (size_t)g * 512;
    *reinterpret_cast<half8 *>(base + (lg * 16 + b) * 8) = half8{hi[0], hi[1], hi[2], hi[3], hi[4], hi[5], hi[6], hi[7]};
    *reinterpret_cast<half8 *>(base + (lg * 16 + 8 + b) * 8) = half8{lo[0], lo[1], lo[2], lo[3], lo[4], lo[5], lo[6], lo[7]};
    if (lg == 0) {
        const float f = b < M ? __builtin_amdgcn_ldexpf(1.0f, -sig) : 0.0f;
        unscale[g * 16 + b] = f;
        unscale[g * 16 + 8 + b] = f;
    }
}

// (q - 8) of the eight nibbles of one word, in the image's k order.
__device__ __forceinline__ half8 unpack_int4(uint32_t w) {
    const half2v off = {(_Float16)1032.0f, (_Float16)1032.0f};
    const half2v p0 = __builtin_bit_cast(half2v, (w & 0x000f000fu) | 0x64006400u) - off;
    const half2v p1 = __builtin_bit_cast(half2v, ((w >> 4) & 0x000f000fu) | 0x64006400u) - off;
    const half2v p2 = __builtin_bit_cast(half2v, ((w >> 8) & 0x000f000fu) | 0x64006400u) - off;
    const half2v p3 = __builtin_bit_cast(half2v, ((w >> 12) & 0x000f000fu) | 0x64006400u) - off;
    return half8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

struct Int4Args {
    const uint32_t *q;
    const uint16_t *scales;
    const _Float16 *img;
    const float *unscale;
    float *out;  // y [M][N] (one split) or partials [splits][M][N]
    int M, N, K, G;
};

// 64 rows x (4 GPW) groups per workgroup; wave w takes groups
// [blockIdx.y 4 GPW + w GPW, + GPW).  A row's GPW groups are GPW * 16
// contiguous bytes: the wave reads them with whole-line 16-byte loads (GPW
// lanes per row) and regroups them through its own LDS slice into the MFMA
// lane order (lane (r, j) takes word j of each group of row r).
template <int GPW>
__global__ __launch_bounds__(256) void int4_gemv_kernel(Int4Args a) {
    __shared__ float red[3][4][4][64];
    __shared__ __attribute__((aligned(16))) uint32_t wl[4][64 * 4 * GPW];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int r0 = blockIdx.x * 64;
    const int g0 = (blockIdx.y * 4 + wave) * GPW;
    const bool active = g0 < a.G;  // a.G is a multiple of GPW
    const int gb = active ? g0 : 0;

    // all loads first: the 64 rows' weight bytes, GPW x fragments and
    // unscale factors, and the scales of this lane's 16 D rows
    constexpr int RPI = 64 / GPW;  // rows per load instruction
    u32x4 wg[GPW];
#pragma unroll
    for (int j = 0; j < GPW; ++j) {
        const int row = j * RPI + lane / GPW;
        wg[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(
            a.q + (size_t)min(r0 + row, a.N - 1) * (a.K / 8) + 4 * (gb + lane % GPW)));
    }
    half8 xb[GPW];
    float f[GPW];
#pragma unroll
    for (int u = 0; u < GPW; ++u) {
        xb[u] = *reinterpret_cast<const half8 *>(a.img + ((size_t)(gb + u) * 64 + lane) * 8);
        f[u] = a.unscale[(gb + u) * 16 + lr];
    }
    u32x4 sv[4][4][GPW / 8];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint16_t *srow = a.scales + (size_t)min(r0 + 16 * t + 4 * lg + i, a.N - 1) * a.G + gb;
#pragma unroll
            for (int h = 0; h < GPW / 8; ++h) sv[t][i][h] = *reinterpret_cast<const u32x4 *>(srow + 8 * h);
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
                const float4v z = {0.0f, 0.0f, 0.0f, 0.0f};
                const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack_int4(w[t][u]), xb[u], z, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t pair = sv[t][i][u >> 3][(u & 7) >> 1];
                    const float s = doe_half_bits_to_float((u & 1) ? (pair >> 16) : pair);
                    acc[t][i] = fmaf(d[i] * f[u], s, acc[t][i]);
                }
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
    // D lane l, tile t: row r0 + 16 t + 4 lg + i, column lr (batch lr % 8; lr / 8: hi / lo)
    const int b = lr & 7;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = acc[t][i] + red[0][t][i][lane] + red[1][t][i][lane] + red[2][t][i][lane];
            v += __shfl_xor(v, 8, 64);
            const int row = r0 + 16 * t + 4 * lg + i;
            if (lr < 8 && b < a.M && row < a.N) a.out[((size_t)blockIdx.y * a.M + b) * a.N + row] = v;
        }
}

__global__ __launch_bounds__(256) void int4_split_sum_kernel(const float *__restrict__ part,
                                                             float *__restrict__ y, int splits,
                                                             int total) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    float s = 0.0f;
    for (int p = 0; p < splits; ++p) s += part[(size_t)p * total + i];
    y[i] = s;
}

std::mutex g_ws_mu;
void *g_ws = nullptr;
size_t g_ws_bytes = 0;
int g_num_cus = 0;

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
        DOE_HIP_CHECK(hipMemsetAsync(y, 0, (size_t)m * n * sizeof(float), st));
        return DOE_OK;
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
    const size_t fac_bytes = (size_t)G * 16 * 4;
    const size_t part_bytes = splits > 1 ? (size_t)splits * m * n * sizeof(float) : 0;
    const size_t need = img_bytes + fac_bytes + part_bytes;
    void *ws;
    {
        std::lock_guard<std::mutex> lk(g_ws_mu);
        if (g_ws_bytes < need) {
            if (g_ws) DOE_HIP_CHECK(hipFree(g_ws));
            g_ws = nullptr;
            g_ws_bytes = 0;
            DOE_HIP_CHECK(hipMalloc(&g_ws, need));
            g_ws_bytes = need;
        }
        ws = g_ws;
    }
    _Float16 *img = (_Float16 *)ws;
    float *unscale = (float *)((char *)ws + img_bytes);
    float *part = (float *)((char *)ws + img_bytes + fac_bytes);
    hipLaunchKernelGGL(int4_x_image_kernel, dim3((unsigned)((G + 7) / 8)), dim3(256), 0, st, x, img, unscale, (int)m,
                       (int)k);
    DOE_LAUNCH_CHECK("int4_x_image_kernel");
    Int4Args a;
    a.q = w_u4;
    a.scales = scales_f16;
    a.img = img;
    a.unscale = unscale;
    a.out = splits > 1 ? part : y;
    a.M = (int)m;
    a.N = (int)n;
    a.K = (int)k;
    a.G = G;
    const dim3 grid((unsigned)row_blocks, (unsigned)splits);
    hipLaunchKernelGGL(int4_gemv_kernel<8>, grid, dim3(256), 0, st, a);
    DOE_LAUNCH_CHECK("int4_gemv_kernel");
    if (splits > 1) {
        const int total = (int)(m * n);
        hipLaunchKernelGGL(int4_split_sum_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, part, y,
                           splits, total);
        DOE_LAUNCH_CHECK("int4_split_sum_kernel");
    }
    return DOE_OK;
}

}  // extern "C"
