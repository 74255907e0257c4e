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
// after a power-of-two scale per batch row), so nothing in the matrix core is
// wasted at M = 8 and the products carry ~22 bits of x.  (q - 8) is exact in
// f16 (OR the nibble into the mantissa of 1024, subtract 1032), each group's
// 16x16 result is scaled by its f16 scale in f32, and the hi/lo halves meet
// in one lane exchange at the end.
//
// A pre-pass writes x as the MFMA's B-operand image ([group][64 lanes][8 f16],
// 1 KB per group, read by every workgroup from L2).  Each wave owns 16 rows
// and a K range; K is split over the grid's y dimension when the rows alone
// do not fill the GPU, and the splits are summed by a small second kernel
// (deterministic order, no atomics).
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
// c / 8: 0 = hi, 1 = lo), x at k = 32 g + 8 (l / 16) + {0, 4, 1, 5, 2, 6, 3, 7}[j].
__global__ __launch_bounds__(256) void int4_x_image_kernel(const float *__restrict__ x,
                                                           _Float16 *__restrict__ img,
                                                           float *__restrict__ unscale, int M,
                                                           int K) {
    const int b = blockIdx.x;
    const int G = K / 32;
    __shared__ float wmax[4];
    __shared__ int ssig;
    int sig = 0;
    if (b < M) {
        float amax = 0.0f;
        for (int k = threadIdx.x; k < K; k += 256) amax = fmaxf(amax, fabsf(x[(size_t)b * K + k]));
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
        if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = amax;
        __syncthreads();
        if (threadIdx.x == 0) {
            const float mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
            int s = 0;
            if (mx > 0.0f && mx <= 3.0e38f) {
                s = 14 - __builtin_amdgcn_frexp_expf(mx);
                s = s < -120 ? -120 : (s > 120 ? 120 : s);
            }
            ssig = s;
            unscale[b] = __builtin_amdgcn_ldexpf(1.0f, -s);
        }
        __syncthreads();
        sig = ssig;
    }
    const float sc = __builtin_amdgcn_ldexpf(1.0f, sig);
    // items: (g, lane group lg, part) -> 8 halves at lane lg*16 + part*8 + b
    for (int it = threadIdx.x; it < G * 8; it += 256) {
        const int g = it >> 3, lg = (it >> 1) & 3, part = it & 1;
        _Float16 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int kk = 32 * g + 8 * lg + ((j & 1) ? 4 + (j >> 1) : (j >> 1));
            float t = b < M ? x[(size_t)b * K + kk] * sc : 0.0f;
            const _Float16 hi = (_Float16)t;
            v[j] = part == 0 ? hi : (_Float16)(t - (float)hi);
        }
        const int lane = lg * 16 + part * 8 + b;
        *reinterpret_cast<half8 *>(img + ((size_t)g * 64 + lane) * 8) =
            half8{v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]};
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
    float *out;  // y [M][N] (splits == 1) or partials [splits][M][N]
    int M, N, K, G, gps;  // gps: groups per split (a multiple of 8)
};

__global__ __launch_bounds__(256) void int4_gemv_kernel(Int4Args a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int r0 = blockIdx.x * 64 + 16 * wave;
    if (r0 >= a.N) return;
    const int g0 = blockIdx.y * a.gps;
    const int g1 = min(a.G, g0 + a.gps);
    const int arow = min(r0 + lr, a.N - 1);
    const uint32_t *qrow = a.q + (size_t)arow * (a.K / 8) + lg;
    const uint16_t *srow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) srow[i] = a.scales + (size_t)min(r0 + 4 * lg + i, a.N - 1) * a.G;
    const _Float16 *ximg = a.img + (size_t)lane * 8;

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int g = g0; g < g1; g += 8) {
        // eight groups at a time: weights, x fragments and the scales of this
        // lane's four D rows, all loads first
        uint32_t w[8];
        half8 xb[8];
        u32x4 sv[4];
#pragma unroll
        for (int u = 0; u < 8; ++u) w[u] = __builtin_nontemporal_load(qrow + 4 * (g + u));
#pragma unroll
        for (int u = 0; u < 8; ++u) xb[u] = *reinterpret_cast<const half8 *>(ximg + (size_t)(g + u) * 512);
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = *reinterpret_cast<const u32x4 *>(srow[i] + g);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float4v z = {0.0f, 0.0f, 0.0f, 0.0f};
            const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack_int4(w[u]), xb[u], z, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t pair = sv[i][u >> 1];
                const float s = doe_half_bits_to_float((u & 1) ? (pair >> 16) : pair);
                acc[i] = fmaf(d[i], s, acc[i]);
            }
        }
    }
    // D lane l: rows r0 + 4 lg + i, column lr (batch lr % 8; lr / 8: hi / lo)
    const int b = lr & 7;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float v = acc[i] + __shfl_xor(acc[i], 8, 64);
        const int row = r0 + 4 * lg + i;
        if (lr < 8 && b < a.M && row < a.N)
            a.out[((size_t)blockIdx.y * a.M + b) * a.N + row] = v * a.unscale[b];
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
    // split K until there are ~4 workgroups per CU, keeping >= 8 groups per split
    int splits = (4 * g_num_cus + row_blocks - 1) / row_blocks;
    const int max_splits = G / 8;
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
    int gps = (G + splits - 1) / splits;
    gps = (gps + 7) / 8 * 8;
    splits = (G + gps - 1) / gps;

    const size_t img_bytes = (size_t)G * 64 * 8 * 2;
    const size_t part_bytes = splits > 1 ? (size_t)splits * m * n * sizeof(float) : 0;
    const size_t need = img_bytes + 64 + part_bytes;
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
    float *part = (float *)((char *)ws + img_bytes + 64);
    hipLaunchKernelGGL(int4_x_image_kernel, dim3(kMaxBatch), dim3(256), 0, st, x, img, unscale, (int)m, (int)k);
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
    a.gps = gps;
    hipLaunchKernelGGL(int4_gemv_kernel, dim3((unsigned)row_blocks, (unsigned)splits), dim3(256), 0, st, a);
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
