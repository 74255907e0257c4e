// q4k_gemm.hip -- Q4_K_M dequant-fused GEMM (prefill) on the gfx950 matrix cores.
//
// C[m][n] = sum_k A[m][k] * dequant(B)[n][k]: A bf16 [M][K] row-major, B the
// row-wise Q4_K_M matrix [N][ceil(K/256) blocks] (bench/tools/doppler_rdrr_q4k.py:
// 128-156), C f32 [M][N] -- the `matmul_q4k` prefill pattern
// (runtime/zig/src/doe_wgsl/emit_csl_classify.zig:287-297; SUMMA with a
// dequantised B tile in emit_csl_matmul_q4k.zig:66-345).
//
// Numerics.  Products run on v_mfma_f32_32x32x16_f16 with f32 accumulation:
//   * A is copied once to f16 by a pre-pass, each row scaled by a power of two
//     2^s_m that puts max|A[m]| just under 2^14; bf16 has 8 significant bits
//     and f16 11, so every element whose scaled magnitude is >= 2^-14 converts
//     exactly (smaller ones carry at least the absolute precision 2^-24 of the
//     row maximum).  The epilogue multiplies row m by 2^-s_m, exactly.
//   * B is dequantised per 64-element chunk into LDS as f16: q is produced
//     exactly with packed-f16 arithmetic ((1024 + q) - 1024 for low nibbles,
//     (64 + q) - 64 for high nibbles, from an OR of the nibble into the
//     mantissa) and w = RN_f16(q * RN_f16(d*sc) - RN_f16(dmin*m)) by one
//     packed fma.  The relative error of w is ~2^-11, far inside the rel-L2
//     1e-3 contract; a bf16 B (8 bits) would sit at ~1.1e-3.
//
// doe_q8_0_gemm_f32 runs the 128 x 128 kernel over Q8_0 rows (34-byte blocks
// of an f16 scale and 32 int8 quants), dequantised to f16 the same way.
//
// Tiling: problems with at least 256 tiles of 256 x 256 use q4k_gemm_pipe_kernel
// (four waves side by side in N, raw B blocks in LDS dequantised per wave,
// software-pipelined); smaller ones use 128 x 128 tiles (2 x 2 waves of 64 x 64)
// with the B chunk dequantised once into LDS.  K runs in steps of one Q4_K
// chunk (64), A and B double-buffered in LDS.  Tiles are ordered in groups of
// 8 M-tiles and each XCD (workgroup id mod 8) gets a contiguous range of that
// order, so the workgroups resident on one XCD share A and B chunks in its L2.
#include "common.h"

#include <math.h>
#include <mutex>

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBK = 64;
constexpr int kLdsRow = kBK + 8;  // halves per LDS row: 144 bytes, b128 reads conflict-free
constexpr int kGroupM = 8;

__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }
__device__ __forceinline__ uint32_t as_u32(half2v v) { return __builtin_bit_cast(uint32_t, v); }

// Scale/min pair of sub-blocks 2*c4 and 2*c4+1 (doppler_rdrr_q4k.py:56-76):
// low byte sub-block 2*c4, high byte 2*c4+1.
__device__ __forceinline__ void scale_min_pair(uint32_t s0, uint32_t s1, uint32_t s2, int c4,
                                               uint32_t &scp, uint32_t &mnp) {
    const int sh = (c4 & 1) * 16;
    if (c4 < 2) {
        scp = (s0 >> sh) & 0x3f3fu;
        mnp = (s1 >> sh) & 0x3f3fu;
    } else {
        scp = ((s2 >> sh) & 0x0f0fu) | ((s0 >> (sh + 2)) & 0x3030u);
        mnp = ((s2 >> (sh + 4)) & 0x0f0fu) | ((s1 >> (sh + 2)) & 0x3030u);
    }
}

// ---------------------------------------------------------------------------
// Pre-pass: A bf16 [M][K] -> f16 [M][Kp] (zero padded to Kp, a multiple of
// 64, or of 256 for the large-tile kernel) scaled by 2^sig[m]; one workgroup
// per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void a_rows_to_f16_kernel(const uint16_t *__restrict__ a,
                                                            _Float16 *__restrict__ a16,
                                                            int *__restrict__ sig, int K, int Kp) {
    const int m = blockIdx.x;
    const uint16_t *row = a + (size_t)m * K;
    _Float16 *out = a16 + (size_t)m * Kp;
    // 16-byte granules of eight elements when the row allows (K % 8 == 0 and an
    // aligned base), several loads in flight per thread; else element by element
    const bool vec = (K & 7) == 0 && ((uintptr_t)row & 15) == 0;
    const int ng = K >> 3;
    float amax = 0.0f;
    if (vec) {
#pragma unroll 4
        for (int gi = threadIdx.x; gi < ng; gi += 256) {
            const u32x4 w = *reinterpret_cast<const u32x4 *>(row + 8 * gi);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                amax = fmaxf(amax, fmaxf(fabsf(__uint_as_float(w[e] << 16)), fabsf(__uint_as_float(w[e] & 0xffff0000u))));
        }
    } else {
        for (int k = threadIdx.x; k < K; k += 256) amax = fmaxf(amax, fabsf(__uint_as_float((uint32_t)row[k] << 16)));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    __shared__ float wmax[4];
    __shared__ int ssig;
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
        sig[m] = s;
    }
    __syncthreads();
    const float scale = __builtin_amdgcn_ldexpf(1.0f, ssig);
    if (vec) {
#pragma unroll 4
        for (int gi = threadIdx.x; gi < (Kp >> 3); gi += 256) {
            u32x4 w = {0u, 0u, 0u, 0u};
            if (gi < ng) w = *reinterpret_cast<const u32x4 *>(row + 8 * gi);
            half8 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                h[2 * e] = (_Float16)(__uint_as_float(w[e] << 16) * scale);
                h[2 * e + 1] = (_Float16)(__uint_as_float(w[e] & 0xffff0000u) * scale);
            }
            *reinterpret_cast<half8 *>(out + 8 * gi) = h;
        }
    } else {
        for (int k = threadIdx.x; k < Kp; k += 256)
            out[k] = k < K ? (_Float16)(__uint_as_float((uint32_t)row[k] << 16) * scale) : (_Float16)0.0f;
    }
}

// The same pre-pass for f32 A: each row scaled by 2^sig[m] (max|A[m]| just
// under 2^14) and rounded once to f16 (11 significant bits).
// f32 rows to f16 with a per-row power-of-two scale (as a_rows_to_f16_kernel
// for bf16), optionally through RMSNorm first (the input_norm /
// post_attn_norm step folded into the projection that consumes it; the
// normalised values are those of the rmsnorm op bit for bit: the same
// per-thread f32 sums of squares over k = t, t + 256, ..., the same
// four-wave sum, inv = 1 / sqrt(ss / K + eps), y = x * inv * (w or 1 + w)).
// R > 0: each thread holds its R elements of the row in registers (K <= 256
// R), so the row is read from memory once; R = 0: the general form re-reads it.
// a16lo != NULL: also the f16 remainder of each scaled value, x * 2^s -
// f16(x * 2^s), so hi + lo carries ~22 bits of the f32 activation.
template <int R, bool NORM>
__global__ __launch_bounds__(256) void a_rows_f32_kernel(const float *__restrict__ a, const float *__restrict__ w,
                                                         float eps, int weight_offset, _Float16 *__restrict__ a16,
                                                         _Float16 *__restrict__ a16lo, int *__restrict__ sig, int K,
                                                         int Kp) {
    const int m = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const float *row = a + (size_t)m * K;
    _Float16 *out = a16 + (size_t)m * Kp;
    __shared__ float sh[4];
    __shared__ int ssig;
    float xv[R > 0 ? R : 1];
    if (R > 0) {
#pragma unroll
        for (int j = 0; j < R; ++j) xv[j] = t + 256 * j < K ? row[t + 256 * j] : 0.0f;
    }
    auto x_at = [&](int j, int k) __attribute__((always_inline)) { return R > 0 ? xv[R > 0 ? j : 0] : row[k]; };
    float inv = 1.0f;
    if (NORM) {
        float ss = 0.0f;
        if (R > 0) {
#pragma unroll
            for (int j = 0; j < R; ++j)
                if (t + 256 * j < K) ss = fmaf(xv[R > 0 ? j : 0], xv[R > 0 ? j : 0], ss);
        } else {
            for (int k = t; k < K; k += 256) ss = fmaf(row[k], row[k], ss);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if (lane == 0) sh[wave] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (int j = 0; j < 4; ++j) tot += sh[j];
        inv = 1.0f / sqrtf(tot / (float)K + eps);
        __syncthreads();  // every thread has read sh
    }
    auto y_at = [&](int j, int k) __attribute__((always_inline)) {
        const float x = x_at(j, k);
        return NORM ? x * inv * (weight_offset ? 1.0f + w[k] : w[k]) : x;
    };
    float amax = 0.0f;
    if (R > 0) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int k = t + 256 * j;
            if (k < K) {
                const float y = y_at(j, k);
                if (NORM) xv[R > 0 ? j : 0] = y;  // keep the normalised value
                amax = fmaxf(amax, fabsf(y));
            }
        }
    } else {
        for (int k = t; k < K; k += 256) amax = fmaxf(amax, fabsf(y_at(0, k)));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    if (lane == 0) sh[wave] = amax;
    __syncthreads();
    if (t == 0) {
        const float mx = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
        int s = 0;
        if (mx > 0.0f && mx <= 3.0e38f) {
            s = 14 - __builtin_amdgcn_frexp_expf(mx);
            s = s < -120 ? -120 : (s > 120 ? 120 : s);
        }
        ssig = s;
        sig[m] = s;
    }
    __syncthreads();
    const float scale = __builtin_amdgcn_ldexpf(1.0f, ssig);
    _Float16 *outlo = a16lo ? a16lo + (size_t)m * Kp : nullptr;
    if (R > 0) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int k = t + 256 * j;
            if (k < K) {
                const float v = xv[R > 0 ? j : 0] * scale;
                const _Float16 h = (_Float16)v;
                out[k] = h;
                if (outlo) outlo[k] = (_Float16)(v - (float)h);
            }
        }
        for (int k = K + t; k < Kp; k += 256) {  // K padding
            out[k] = (_Float16)0.0f;
            if (outlo) outlo[k] = (_Float16)0.0f;
        }
    } else {
        for (int k = t; k < Kp; k += 256) {
            const float v = k < K ? y_at(0, k) * scale : 0.0f;
            const _Float16 h = (_Float16)v;
            out[k] = h;
            if (outlo) outlo[k] = (_Float16)(v - (float)h);
        }
    }
}

// Launch of the f32 pre-pass: the register form up to K = 256 x 48.
void launch_a_rows_f32(const float *a, const float *w, float eps, int offset, _Float16 *a16, _Float16 *a16lo,
                       int *sig, int64_t m, int64_t k, int64_t kp, hipStream_t st) {
    const int r = (int)((k + 255) / 256);
#define DOE_A_ROWS(R)                                                                                          \
    do {                                                                                                       \
        if (w)                                                                                                 \
            hipLaunchKernelGGL((a_rows_f32_kernel<R, true>), dim3((unsigned)m), dim3(256), 0, st, a, w, eps, offset, \
                               a16, a16lo, sig, (int)k, (int)kp);                                              \
        else                                                                                                   \
            hipLaunchKernelGGL((a_rows_f32_kernel<R, false>), dim3((unsigned)m), dim3(256), 0, st, a, w, eps, offset, \
                               a16, a16lo, sig, (int)k, (int)kp);                                              \
    } while (0)
    if (r <= 4) DOE_A_ROWS(4);
    else if (r <= 12) DOE_A_ROWS(12);
    else if (r <= 24) DOE_A_ROWS(24);
    else if (r <= 48) DOE_A_ROWS(48);
    else DOE_A_ROWS(0);
#undef DOE_A_ROWS
}

// ---------------------------------------------------------------------------
// GEMM.
// ---------------------------------------------------------------------------
struct GemmArgs {
    const _Float16 *a16;
    const _Float16 *a16lo;  // the f32-accurate kernel: the f16 remainders of A
    const int *sig;
    const uint8_t *b;
    float *c;
    int M, N, Kp, nb, nchunk, tiles_m, tiles_n;
    // K split of the small-tile kernel (gridDim.y > 1): split y runs chunks
    // [y kps, (y + 1) kps) and writes its partial tile to part + y M N
    float *part;
    int kps;
};

// Four halves from the low nibbles and four from the high nibbles of one
// nibble dword (bytes b0..b3 = consecutive k), each as exact f16 values
// q * dsc - dmm rounded once.
__device__ __forceinline__ void dequant_dword(uint32_t w, half2v dsc_lo, half2v ndmm_lo, half2v dsc_hi,
                                              half2v ndmm_hi, uint32_t *lo, uint32_t *hi) {
    // t0 = [b0, 0, b1, 0], t1 = [b2, 0, b3, 0]
    const uint32_t t0 = __builtin_amdgcn_perm(0u, w, 0x0c010c00u);
    const uint32_t t1 = __builtin_amdgcn_perm(0u, w, 0x0c030c02u);
    const half2v k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    const half2v k64 = {(_Float16)64.0f, (_Float16)64.0f};
    const half2v ql0 = as_h2((t0 & 0x000f000fu) | 0x64006400u) - k1024;
    const half2v ql1 = as_h2((t1 & 0x000f000fu) | 0x64006400u) - k1024;
    const half2v qh0 = as_h2((t0 & 0x00f000f0u) | 0x54005400u) - k64;
    const half2v qh1 = as_h2((t1 & 0x00f000f0u) | 0x54005400u) - k64;
    lo[0] = as_u32(__builtin_elementwise_fma(ql0, dsc_lo, ndmm_lo));
    lo[1] = as_u32(__builtin_elementwise_fma(ql1, dsc_lo, ndmm_lo));
    hi[0] = as_u32(__builtin_elementwise_fma(qh0, dsc_hi, ndmm_hi));
    hi[1] = as_u32(__builtin_elementwise_fma(qh1, dsc_hi, ndmm_hi));
}

// TM x TN 32x32 accumulators per wave, 2 x 2 waves: a (64 TM) x (64 TN) tile.
// FMT 0: B is row-wise Q4_K_M; FMT 1: B is row-wise Q8_0 (nb = ceil(K / 32)
// blocks of 34 bytes: f16 d, 32 int8 q, weight d * q; blocks only 2-byte
// aligned): the two threads of a B row each dequantise one block of the
// chunk, w = RN_f16(d * q) (d * q is exact in f32).
template <int TM, int TN, int FMT>
__global__ __launch_bounds__(256) void quant_gemm_kernel(GemmArgs g) {
    constexpr int BM = 64 * TM, BN = 64 * TN;
    constexpr int GA = BM / 32;      // 16-byte A granules per thread per chunk
    constexpr int TPR = 256 / BN;    // threads per B row (1 or 2)
    constexpr int NBY = 32 / TPR;    // nibble bytes per thread per chunk (32 or 16)
    constexpr int NQ = NBY / 16;     // 16-byte nibble loads per thread
    static_assert(FMT == 0 || TPR == 2, "Q8_0 staging: two threads per B row, one block each");
    __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * kLdsRow];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * kLdsRow];
    // 2^-sig of the tile's rows: the epilogue's stores never wait on a
    // global load (cout may alias sig as far as the compiler knows, so each
    // row's load would otherwise wait for the stores before it)
    __shared__ float rowscale[BM];

    // tile order: XCD-contiguous ranges of an M-grouped raster
    const int T = g.tiles_m * g.tiles_n;
    int t = blockIdx.x;
    if ((T & 7) == 0) t = (blockIdx.x & 7) * (T >> 3) + (blockIdx.x >> 3);
    const int per_group = kGroupM * g.tiles_n;
    const int grp = t / per_group;
    const int first_m = grp * kGroupM;
    const int gsize = min(kGroupM, g.tiles_m - first_m);
    const int within = t - grp * per_group;
    const int tm = first_m + within % gsize;
    const int tn = within / gsize;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // global -> register staging assignments
    // A: granule gi = tid + 256 i: row gi >> 3, col (gi & 7) * 8
    // B: row tid / TPR, nibble bytes [boff, boff + NBY) of the chunk
    const int brow = tid / TPR, boff = (tid % TPR) * NBY;
    const uint8_t *brow_ptr = g.b + (size_t)min(n0 + brow, g.N - 1) * g.nb * DOE_Q4K_BLOCK_BYTES;
    // Q8_0: buffer loads over the whole matrix, its size rounded up to a whole
    // dword (the range check is per dword: the last block's last quants share
    // a dword with up to two bytes past the matrix, which a 4-byte-aligned
    // weight keeps on the same page); a block's 36-byte dword-aligned window
    // read from an offset past the end reads zero
    const __amdgpu_buffer_rsrc_t b8rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)g.b, (short)0, FMT == 1 ? (int)(((uint32_t)g.N * (uint32_t)g.nb * 34u + 3u) & ~3u) : 0, 0x00020000);
    const uint32_t b8row = (uint32_t)min(n0 + brow, g.N - 1) * (uint32_t)g.nb;
    const _Float16 *arow_ptr[GA];
#pragma unroll
    for (int i = 0; i < GA; ++i) {
        const int gi = tid + 256 * i;
        arow_ptr[i] = g.a16 + (size_t)min(m0 + (gi >> 3), g.M - 1) * g.Kp + (gi & 7) * 8;
    }

    u32x4 ra[GA], rh, rq[NQ];
    u32x4 r8a, r8b;  // Q8_0: the block's dword-aligned 36-byte window
    uint32_t r8c, r8sh;
    // (macros, not lambdas: the staging arrays must stay in registers)
#define DOE_GEMM_LOAD_CHUNK(KC)                                                                        \
    do {                                                                                               \
        _Pragma("unroll") for (int i = 0; i < GA; ++i)                                                 \
            ra[i] = *reinterpret_cast<const u32x4 *>(arow_ptr[i] + (KC) * kBK);                        \
        if constexpr (FMT == 0) {                                                                      \
            const uint8_t *blk_ = brow_ptr + (size_t)((KC) >> 2) * DOE_Q4K_BLOCK_BYTES;                \
            rh = *reinterpret_cast<const u32x4 *>(blk_);                                               \
            _Pragma("unroll") for (int j = 0; j < NQ; ++j)                                             \
                rq[j] = *reinterpret_cast<const u32x4 *>(blk_ + 16 + 32 * ((KC) & 3) + boff + 16 * j); \
        } else {                                                                                       \
            const int bi_ = 2 * (KC) + (tid & 1);                                                      \
            const uint32_t o_ = bi_ < g.nb ? (b8row + (uint32_t)bi_) * 34u : 0x80000000u;              \
            const uint32_t al_ = o_ & ~3u;                                                             \
            r8a = __builtin_amdgcn_raw_buffer_load_b128(b8rsrc, al_, 0, 0);                           \
            r8b = __builtin_amdgcn_raw_buffer_load_b128(b8rsrc, al_ + 16u, 0, 0);                     \
            r8c = __builtin_amdgcn_raw_buffer_load_b32(b8rsrc, al_ + 32u, 0, 0);                      \
            r8sh = o_ & 2u;                                                                            \
        }                                                                                              \
    } while (0)
#define DOE_GEMM_STORE_CHUNK(BUF, KC)                                                                  \
    do {                                                                                               \
        _Pragma("unroll") for (int i = 0; i < GA; ++i) {                                               \
            const int gi = tid + 256 * i;                                                              \
            *reinterpret_cast<u32x4 *>(&As[BUF][(gi >> 3) * kLdsRow + (gi & 7) * 8]) = ra[i];          \
        }                                                                                              \
        if constexpr (FMT == 1) {                                                                      \
            const uint32_t dw_[9] = {r8a.x, r8a.y, r8a.z, r8a.w, r8b.x, r8b.y, r8b.z, r8b.w, r8c};     \
            const uint32_t sh_ = r8sh << 3; /* the block starts at byte 0 or 2 of the window */       \
            const uint32_t sel_ = sh_ ? 0x07060504u : 0x05040302u;                                     \
            const float d8_ = doe_half_bits_to_float(__builtin_amdgcn_ubfe(dw_[0], sh_, 16));          \
            uint32_t hv_[16];                                                                          \
            _Pragma("unroll") for (int j = 0; j < 8; ++j) {                                            \
                const uint32_t u_ = __builtin_amdgcn_perm(dw_[j + 1], dw_[j], sel_);                   \
                const half2v w01 = {(_Float16)(d8_ * (float)(int8_t)(u_ & 0xffu)),                     \
                                    (_Float16)(d8_ * (float)(int8_t)((u_ >> 8) & 0xffu))};             \
                const half2v w23 = {(_Float16)(d8_ * (float)(int8_t)((u_ >> 16) & 0xffu)),             \
                                    (_Float16)(d8_ * (float)(int8_t)(u_ >> 24))};                      \
                hv_[2 * j] = as_u32(w01);                                                              \
                hv_[2 * j + 1] = as_u32(w23);                                                          \
            }                                                                                          \
            _Float16 *bl8_ = &Bs[BUF][brow * kLdsRow + (tid & 1) * 32];                                \
            _Pragma("unroll") for (int j = 0; j < 4; ++j)                                              \
                *reinterpret_cast<u32x4 *>(bl8_ + 8 * j) =                                             \
                    u32x4{hv_[4 * j], hv_[4 * j + 1], hv_[4 * j + 2], hv_[4 * j + 3]};                 \
            break;                                                                                     \
        }                                                                                              \
        uint32_t scp_, mnp_;                                                                           \
        scale_min_pair(rh.y, rh.z, rh.w, (KC) & 3, scp_, mnp_);                                        \
        const float d_ = doe_half_bits_to_float(rh.x), dmin_ = doe_half_bits_to_float(rh.x >> 16);     \
        const _Float16 dsl_ = (_Float16)(d_ * (float)(scp_ & 0xffu));                                  \
        const _Float16 dsh_ = (_Float16)(d_ * (float)(scp_ >> 8));                                     \
        const _Float16 dml_ = (_Float16)(-(dmin_ * (float)(mnp_ & 0xffu)));                            \
        const _Float16 dmh_ = (_Float16)(-(dmin_ * (float)(mnp_ >> 8)));                               \
        const half2v dsc_lo = {dsl_, dsl_}, dsc_hi = {dsh_, dsh_}, ndmm_lo = {dml_, dml_},             \
                     ndmm_hi = {dmh_, dmh_};                                                           \
        _Pragma("unroll") for (int j = 0; j < NQ; ++j) {                                               \
            uint32_t lo[8], hi[8];                                                                     \
            dequant_dword(rq[j].x, dsc_lo, ndmm_lo, dsc_hi, ndmm_hi, lo + 0, hi + 0);                  \
            dequant_dword(rq[j].y, dsc_lo, ndmm_lo, dsc_hi, ndmm_hi, lo + 2, hi + 2);                  \
            dequant_dword(rq[j].z, dsc_lo, ndmm_lo, dsc_hi, ndmm_hi, lo + 4, hi + 4);                  \
            dequant_dword(rq[j].w, dsc_lo, ndmm_lo, dsc_hi, ndmm_hi, lo + 6, hi + 6);                  \
            _Float16 *bl = &Bs[BUF][brow * kLdsRow + boff + 16 * j];                                   \
            *reinterpret_cast<u32x4 *>(bl) = u32x4{lo[0], lo[1], lo[2], lo[3]};                        \
            *reinterpret_cast<u32x4 *>(bl + 8) = u32x4{lo[4], lo[5], lo[6], lo[7]};                    \
            *reinterpret_cast<u32x4 *>(bl + 32) = u32x4{hi[0], hi[1], hi[2], hi[3]};                   \
            *reinterpret_cast<u32x4 *>(bl + 40) = u32x4{hi[4], hi[5], hi[6], hi[7]};                   \
        }                                                                                              \
    } while (0)

    float16v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    for (int r = tid; r < BM; r += 256) rowscale[r] = __builtin_amdgcn_ldexpf(1.0f, -g.sig[min(m0 + r, g.M - 1)]);
    const int kc0 = (int)blockIdx.y * g.kps, kc1 = min(g.nchunk, kc0 + g.kps);
    float *cout = gridDim.y > 1 ? g.part + (size_t)blockIdx.y * g.M * g.N : g.c;
    DOE_GEMM_LOAD_CHUNK(kc0);
    DOE_GEMM_STORE_CHUNK(0, kc0);
    __syncthreads();
    const int lr = lane & 31, lk = 8 * (lane >> 5);
    for (int kc = kc0; kc < kc1; ++kc) {
        const int buf = (kc - kc0) & 1;
        if (kc + 1 < kc1) DOE_GEMM_LOAD_CHUNK(kc + 1);
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks) {
            half8 af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *reinterpret_cast<const half8 *>(&As[buf][(wm * 32 * TM + i * 32 + lr) * kLdsRow + ks * 16 + lk]);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bf[j] = *reinterpret_cast<const half8 *>(&Bs[buf][(wn * 32 * TN + j * 32 + lr) * kLdsRow + ks * 16 + lk]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kc + 1 < kc1) DOE_GEMM_STORE_CHUNK(buf ^ 1, kc + 1);
        __syncthreads();
    }
#undef DOE_GEMM_LOAD_CHUNK
#undef DOE_GEMM_STORE_CHUNK

    // epilogue: D lane l, r: row (r%4) + 8(r/4) + 4(l/32), column l%32
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int mt = wm * 32 * TM + i * 32 + (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5);
            const int m = m0 + mt;
            if (m >= g.M) continue;
            const float us = rowscale[mt];
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int n = n0 + wn * 32 * TN + j * 32 + lr;
                if (n < g.N) cout[(size_t)m * g.N + n] = acc[i][j][r] * us;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// f32-accurate GEMM for f32 activations (the decoder's batched prompt): the
// 128 x 128 tile of quant_gemm_kernel with both operands carried as f16 hi +
// lo pairs.  A = a_hi + a_lo from the pre-pass (~22 bits of the scaled f32
// row); B = b_hi + b_lo from the f32 dequantised weight -- Q4_K: fmaf(d sc,
// q, -(dmin m)), the canonical decode rounded once to f32; Q8_0: d q, exact
// in f32 -- (b_hi + b_lo is that f32 weight to ~22 bits).  Each 16-k step
// runs a_hi b_hi + a_lo b_hi + a_hi b_lo on the matrix cores (every product
// exact in f32, f32 accumulation; the dropped a_lo b_lo is ~2^-22 of the
// product), so the result sits at f32-GEMV accuracy instead of the ~2^-12
// of one f16 rounding per operand.  K runs in 32-element chunks (one Q4_K
// sub-block or one Q8_0 block per row), four f16 tiles double-buffered in
// LDS (73.7 KB: two workgroups per CU).
// ---------------------------------------------------------------------------
constexpr int kXBK = 32;        // K per chunk
constexpr int kXLdsRow = 36;    // halves per LDS row: 72 bytes (73.7 KB in all: two workgroups per CU)

template <int FMT>
__global__ __launch_bounds__(256) void quant_gemm_exact_kernel(GemmArgs g) {
    constexpr int TM = 2, TN = 2, BM = 128, BN = 128;
    __shared__ __attribute__((aligned(16))) _Float16 Ah[2][BM * kXLdsRow];
    __shared__ __attribute__((aligned(16))) _Float16 Al[2][BM * kXLdsRow];
    __shared__ __attribute__((aligned(16))) _Float16 Bh[2][BN * kXLdsRow];
    __shared__ __attribute__((aligned(16))) _Float16 Bl[2][BN * kXLdsRow];
    __shared__ float rowscale[BM];

    // tile order: XCD-contiguous ranges of an M-grouped raster (as quant_gemm_kernel)
    const int T = g.tiles_m * g.tiles_n;
    int t = blockIdx.x;
    if ((T & 7) == 0) t = (blockIdx.x & 7) * (T >> 3) + (blockIdx.x >> 3);
    const int per_group = kGroupM * g.tiles_n;
    const int grp = t / per_group;
    const int first_m = grp * kGroupM;
    const int gsize = min(kGroupM, g.tiles_m - first_m);
    const int within = t - grp * per_group;
    const int tm = first_m + within % gsize;
    const int tn = within / gsize;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // A: thread t stages granules t and t + 256 (row gi >> 2, halves (gi & 3) * 8) of hi and lo
    // B: thread t stages row t >> 1, elements (t & 1) * 16 .. + 15 of the chunk
    const int brow = tid >> 1, bhalf = tid & 1;
    const int nrow = min(n0 + brow, g.N - 1);
    const _Float16 *ah_ptr[2], *al_ptr[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int gi = tid + 256 * i;
        const size_t off = (size_t)min(m0 + (gi >> 2), g.M - 1) * g.Kp + (gi & 3) * 8;
        ah_ptr[i] = g.a16 + off;
        al_ptr[i] = g.a16lo + off;
    }
    const uint8_t *brow_ptr = g.b + (size_t)nrow * g.nb * DOE_Q4K_BLOCK_BYTES;
    const __amdgpu_buffer_rsrc_t b8rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)g.b, (short)0, FMT == 1 ? (int)(((uint32_t)g.N * (uint32_t)g.nb * 34u + 3u) & ~3u) : 0, 0x00020000);
    const uint32_t b8row = (uint32_t)nrow * (uint32_t)g.nb;

    u32x4 rah[2], ral[2], rh, rq, r8a, r8b;
    uint32_t r8c = 0, r8sh = 0;
#define DOE_XGEMM_LOAD(KC)                                                                               \
    do {                                                                                                 \
        _Pragma("unroll") for (int i = 0; i < 2; ++i) {                                                  \
            rah[i] = *reinterpret_cast<const u32x4 *>(ah_ptr[i] + (KC) * kXBK);                          \
            ral[i] = *reinterpret_cast<const u32x4 *>(al_ptr[i] + (KC) * kXBK);                          \
        }                                                                                                \
        if constexpr (FMT == 0) {                                                                        \
            /* sub-block KC % 8 of block KC / 8: nibble bytes of chunk (KC % 8) / 2, low or high */      \
            const uint8_t *blk_ = brow_ptr + (size_t)((KC) >> 3) * DOE_Q4K_BLOCK_BYTES;                  \
            rh = *reinterpret_cast<const u32x4 *>(blk_);                                                 \
            rq = *reinterpret_cast<const u32x4 *>(blk_ + 16 + 32 * (((KC) & 7) >> 1) + 16 * bhalf);      \
        } else {                                                                                         \
            const uint32_t o_ = (KC) < g.nb ? (b8row + (uint32_t)(KC)) * 34u : 0x80000000u;              \
            const uint32_t al_ = o_ & ~3u;                                                               \
            r8a = __builtin_amdgcn_raw_buffer_load_b128(b8rsrc, al_, 0, 0);                             \
            r8b = __builtin_amdgcn_raw_buffer_load_b128(b8rsrc, al_ + 16u, 0, 0);                       \
            r8c = __builtin_amdgcn_raw_buffer_load_b32(b8rsrc, al_ + 32u, 0, 0);                        \
            r8sh = o_ & 2u;                                                                              \
        }                                                                                                \
    } while (0)
#define DOE_XGEMM_STORE(BUF, KC)                                                                         \
    do {                                                                                                 \
        _Pragma("unroll") for (int i = 0; i < 2; ++i) {                                                  \
            const int gi = tid + 256 * i;                                                                \
            const int lo_ = (gi >> 2) * kXLdsRow + (gi & 3) * 8;                                         \
            *reinterpret_cast<u32x4 *>(&Ah[BUF][lo_]) = rah[i];                                          \
            *reinterpret_cast<u32x4 *>(&Al[BUF][lo_]) = ral[i];                                          \
        }                                                                                                \
        float w_[16];                                                                                    \
        if constexpr (FMT == 0) {                                                                        \
            const int sb_ = (KC) & 7, c4_ = sb_ >> 1;                                                    \
            uint32_t scp_, mnp_;                                                                         \
            scale_min_pair(rh.y, rh.z, rh.w, c4_, scp_, mnp_);                                           \
            const int sh8_ = (sb_ & 1) * 8;                                                              \
            const float dsc_ = doe_half_bits_to_float(rh.x) * (float)((scp_ >> sh8_) & 0xffu);           \
            const float dmm_ = doe_half_bits_to_float(rh.x >> 16) * (float)((mnp_ >> sh8_) & 0xffu);     \
            const int nsh_ = (sb_ & 1) * 4;                                                              \
            _Pragma("unroll") for (int j = 0; j < 16; ++j) {                                             \
                const uint32_t byte_ = (rq[j >> 2] >> (8 * (j & 3))) & 0xffu;                            \
                w_[j] = fmaf(dsc_, (float)((byte_ >> nsh_) & 15u), -dmm_);                               \
            }                                                                                            \
        } else {                                                                                         \
            const uint32_t dw_[9] = {r8a.x, r8a.y, r8a.z, r8a.w, r8b.x, r8b.y, r8b.z, r8b.w, r8c};       \
            const uint32_t sh_ = r8sh << 3; /* the block starts at byte 0 or 2 of the window */         \
            const uint32_t sel_ = sh_ ? 0x07060504u : 0x05040302u;                                       \
            const float d8_ = doe_half_bits_to_float(__builtin_amdgcn_ubfe(dw_[0], sh_, 16));            \
            _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                              \
                const uint32_t u_ = __builtin_amdgcn_perm(dw_[4 * bhalf + j + 1], dw_[4 * bhalf + j], sel_); \
                _Pragma("unroll") for (int e = 0; e < 4; ++e)                                            \
                    w_[4 * j + e] = d8_ * (float)(int8_t)((u_ >> (8 * e)) & 0xffu);                      \
            }                                                                                            \
        }                                                                                                \
        uint32_t hv_[8], lv_[8];                                                                         \
        _Pragma("unroll") for (int j = 0; j < 8; ++j) {                                                  \
            const _Float16 h0 = (_Float16)w_[2 * j], h1 = (_Float16)w_[2 * j + 1];                       \
            const _Float16 l0 = (_Float16)(w_[2 * j] - (float)h0), l1 = (_Float16)(w_[2 * j + 1] - (float)h1); \
            hv_[j] = as_u32(half2v{h0, h1});                                                             \
            lv_[j] = as_u32(half2v{l0, l1});                                                             \
        }                                                                                                \
        const int bo_ = brow * kXLdsRow + 16 * bhalf;                                                    \
        *reinterpret_cast<u32x4 *>(&Bh[BUF][bo_]) = u32x4{hv_[0], hv_[1], hv_[2], hv_[3]};               \
        *reinterpret_cast<u32x4 *>(&Bh[BUF][bo_ + 8]) = u32x4{hv_[4], hv_[5], hv_[6], hv_[7]};           \
        *reinterpret_cast<u32x4 *>(&Bl[BUF][bo_]) = u32x4{lv_[0], lv_[1], lv_[2], lv_[3]};               \
        *reinterpret_cast<u32x4 *>(&Bl[BUF][bo_ + 8]) = u32x4{lv_[4], lv_[5], lv_[6], lv_[7]};           \
    } while (0)

    float16v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    for (int r = tid; r < BM; r += 256) rowscale[r] = __builtin_amdgcn_ldexpf(1.0f, -g.sig[min(m0 + r, g.M - 1)]);
    const int kc0 = (int)blockIdx.y * g.kps, kc1 = min(g.nchunk, kc0 + g.kps);
    float *cout = gridDim.y > 1 ? g.part + (size_t)blockIdx.y * g.M * g.N : g.c;
    DOE_XGEMM_LOAD(kc0);
    DOE_XGEMM_STORE(0, kc0);
    __syncthreads();
    const int lr = lane & 31, lk = 8 * (lane >> 5);
    for (int kc = kc0; kc < kc1; ++kc) {
        const int buf = (kc - kc0) & 1;
        if (kc + 1 < kc1) DOE_XGEMM_LOAD(kc + 1);
#pragma unroll
        for (int ks = 0; ks < kXBK / 16; ++ks) {
            half8 ah[TM], al[TM], bh[TN], bl[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int o = (wm * 32 * TM + i * 32 + lr) * kXLdsRow + ks * 16 + lk;
                ah[i] = *reinterpret_cast<const half8 *>(&Ah[buf][o]);
                al[i] = *reinterpret_cast<const half8 *>(&Al[buf][o]);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int o = (wn * 32 * TN + j * 32 + lr) * kXLdsRow + ks * 16 + lk;
                bh[j] = *reinterpret_cast<const half8 *>(&Bh[buf][o]);
                bl[j] = *reinterpret_cast<const half8 *>(&Bl[buf][o]);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bh[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bh[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bl[j], acc[i][j], 0, 0, 0);
                }
        }
        if (kc + 1 < kc1) DOE_XGEMM_STORE(buf ^ 1, kc + 1);
        __syncthreads();
    }
#undef DOE_XGEMM_LOAD
#undef DOE_XGEMM_STORE

    // epilogue: D lane l, r: row (r%4) + 8(r/4) + 4(l/32), column l%32
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int mt = wm * 32 * TM + i * 32 + (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5);
            const int m = m0 + mt;
            if (m >= g.M) continue;
            const float us = rowscale[mt];
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int n = n0 + wn * 32 * TN + j * 32 + lr;
                if (n < g.N) cout[(size_t)m * g.N + n] = acc[i][j][r] * us;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Large-problem GEMM: 256 (M) x 256 (N) tile per 256-thread workgroup, the
// four waves side by side in N (wave w owns columns 64w..64w+63 for all 256
// rows: 8 x 2 accumulators of v_mfma_f32_32x32x16_f16).  B is staged raw:
// each Q4_K block (144 bytes) of the tile's 256 rows is loaded once per 256 K
// with line-contiguous 16-byte granules and kept in LDS, and each wave
// dequantises its MFMA B operands straight from those bytes (8 nibbles -> 8
// f16 per lane per 16-k step).  A is staged as f16 per 64-element chunk.
// Every latency is kept off the MFMA stream (one wave per SIMD issues in
// order, so anything it waits on idles the matrix core):
//   * the MFMA operands of 16-k step s + 1 (eight A fragments, two raw B
//     granules, dequantised in registers) are read and converted while the
//     sixteen MFMAs of step s run, interleaved one LDS read or a few VALU
//     operations per MFMA;
//   * A chunk c + 1 is written to LDS at the start of chunk c (its global
//     loads were issued one chunk earlier) and B block b + 1 at the start of
//     block b (loads four chunks earlier), so one barrier per chunk, waiting
//     on LDS only, separates the writes from the next chunk's reads;
//   * global loads are buffer loads over the tile's rows with 32-bit offsets:
//     rows past M or N read as zero, no per-granule 64-bit pointers;
//   * the four chunks of a Q4_K block are unrolled, so buffer parities and the
//     sub-block scale selection are compile-time constants;
//   * the row unscaling factors sit in LDS, so the epilogue's stores never
//     wait on a global load.
// A is the f16 copy padded to a whole number of Q4_K blocks (Kp = 256 nb).
// ---------------------------------------------------------------------------
constexpr int kRawRow = 152;  // bytes per raw B row: 144 + 8 pad, conflict-free b64 reads

// Eight f16 operands from 8 nibble bytes (two dwords): low (HI = false) or
// high nibbles, w = RN_f16(q * dsc - dmm).
template <bool HI>
__device__ __forceinline__ half8 dequant8(uint32_t w0, uint32_t w1, half2v dsc, half2v ndmm) {
    const half2v bias = HI ? half2v{(_Float16)64.0f, (_Float16)64.0f} : half2v{(_Float16)1024.0f, (_Float16)1024.0f};
    const uint32_t mask = HI ? 0x00f000f0u : 0x000f000fu;
    const uint32_t magic = HI ? 0x54005400u : 0x64006400u;
    const uint32_t t[4] = {__builtin_amdgcn_perm(0u, w0, 0x0c010c00u), __builtin_amdgcn_perm(0u, w0, 0x0c030c02u),
                           __builtin_amdgcn_perm(0u, w1, 0x0c010c00u), __builtin_amdgcn_perm(0u, w1, 0x0c030c02u)};
    half8 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const half2v q = as_h2((t[e] & mask) | magic) - bias;
        const half2v v = __builtin_elementwise_fma(q, dsc, ndmm);
        r[2 * e] = v[0];
        r[2 * e + 1] = v[1];
    }
    return r;
}

constexpr int kBufFlags = 0x00020000;  // raw buffer, 32-bit data format

// Scales of chunk c4's two sub-blocks for one B row from its 16 header bytes.
template <int C4>
__device__ __forceinline__ void chunk_scales(const u32x4 &h, half2v &dsc_lo, half2v &ndmm_lo, half2v &dsc_hi,
                                             half2v &ndmm_hi) {
    uint32_t scp, mnp;
    scale_min_pair(h.y, h.z, h.w, C4, scp, mnp);
    const float d = doe_half_bits_to_float(h.x), dmin = doe_half_bits_to_float(h.x >> 16);
    const _Float16 s0 = (_Float16)(d * (float)(scp & 0xffu)), s1 = (_Float16)(d * (float)(scp >> 8));
    const _Float16 z0 = (_Float16)(-(dmin * (float)(mnp & 0xffu)));
    const _Float16 z1 = (_Float16)(-(dmin * (float)(mnp >> 8)));
    dsc_lo = half2v{s0, s0};
    dsc_hi = half2v{s1, s1};
    ndmm_lo = half2v{z0, z0};
    ndmm_hi = half2v{z1, z1};
}

// Barrier for LDS hand-offs only: outstanding global loads stay in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__global__ __launch_bounds__(256) void q4k_gemm_pipe_kernel(GemmArgs g) {
    constexpr int BM = 256, BN = 256;
    __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * kLdsRow];
    __shared__ __attribute__((aligned(16))) uint8_t Braw[2][BN * kRawRow];
    __shared__ float rowscale[BM];  // 2^-sig of the tile's rows (exact unscaling)

    const int T = g.tiles_m * g.tiles_n;
    int t = blockIdx.x;
    if ((T & 7) == 0) t = (blockIdx.x & 7) * (T >> 3) + (blockIdx.x >> 3);
    const int per_group = kGroupM * g.tiles_n;
    const int grp = t / per_group;
    const int first_m = grp * kGroupM;
    const int gsize = min(kGroupM, g.tiles_m - first_m);
    const int within = t - grp * per_group;
    const int m0 = (first_m + within % gsize) * BM;
    const int n0 = (within / gsize) * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 31, lk = 8 * (lane >> 5);

    const uint32_t a_stride = (uint32_t)g.Kp * 2u;
    const uint32_t brow_bytes = (uint32_t)g.nb * DOE_Q4K_BLOCK_BYTES;
    const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(g.a16 + (size_t)m0 * g.Kp), (short)0, (int)((uint32_t)min(BM, g.M - m0) * a_stride), kBufFlags);
    const __amdgpu_buffer_rsrc_t brsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(g.b + (size_t)n0 * brow_bytes), (short)0, (int)((uint32_t)min(BN, g.N - n0) * brow_bytes), kBufFlags);
    // A granule i: row (tid >> 3) + 32 i, bytes 16 (tid & 7) of the chunk
    const uint32_t a_voff = (uint32_t)(tid >> 3) * a_stride + (uint32_t)(tid & 7) * 16u;
    const int a_lds = (tid >> 3) * kLdsRow + (tid & 7) * 8;

    u32x4 ra[8], rb[9];
#define DOE_PIPE_LOAD_A(KC)                                                                            \
    _Pragma("unroll") for (int i = 0; i < 8; ++i) ra[i] = __builtin_amdgcn_raw_buffer_load_b128(         \
        arsrc, a_voff + (uint32_t)i * 32u * a_stride, (KC) * (kBK * 2), 0)
#define DOE_PIPE_STORE_A(BUF)                                                                          \
    _Pragma("unroll") for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x4 *>(&As[BUF][a_lds + i * 32 * kLdsRow]) = ra[i]
    // B granule i: gi = tid + 256 i -> row gi / 9, 16-byte piece gi % 9
#define DOE_PIPE_LOAD_B(BLK)                                                                           \
    _Pragma("unroll") for (int i = 0; i < 9; ++i) {                                                    \
        const int gi_ = tid + 256 * i, row_ = gi_ / 9;                                                 \
        rb[i] = __builtin_amdgcn_raw_buffer_load_b128(                                                 \
            brsrc, (uint32_t)row_ * brow_bytes + (uint32_t)(gi_ - 9 * row_) * 16u, (BLK) * DOE_Q4K_BLOCK_BYTES, 0); \
    }
#define DOE_PIPE_STORE_B(BUF)                                                                          \
    _Pragma("unroll") for (int i = 0; i < 9; ++i) {                                                    \
        const int gi_ = tid + 256 * i, row_ = gi_ / 9;                                                 \
        u32x2 *d_ = reinterpret_cast<u32x2 *>(&Braw[BUF][row_ * kRawRow + (gi_ - 9 * row_) * 16]);     \
        d_[0] = u32x2{rb[i].x, rb[i].y};                                                               \
        d_[1] = u32x2{rb[i].z, rb[i].w};                                                               \
    }

    float16v acc[8][2];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // this lane's two B rows within the tile
    int brow[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) brow[j] = (wave * 64 + j * 32 + lr) * kRawRow;
    const int afrag = lr * kLdsRow + lk;

    const int sig_row = g.sig[min(m0 + tid, g.M - 1)];
    DOE_PIPE_LOAD_A(0);
    DOE_PIPE_LOAD_B(0);
    rowscale[tid] = __builtin_amdgcn_ldexpf(1.0f, -sig_row);
    DOE_PIPE_STORE_A(0);
    DOE_PIPE_STORE_B(0);
    DOE_PIPE_LOAD_A(min(1, g.nchunk - 1));
    DOE_PIPE_LOAD_B(min(1, g.nb - 1));
    lds_barrier();

    // operands of step (chunk 0, k-step 0)
    u32x4 hdr[2];
    half2v dsc[2][2], ndmm[2][2];
    half8 af[2][8], bf[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const u32x2 h01 = *reinterpret_cast<const u32x2 *>(&Braw[0][brow[j]]);
        const u32x2 h23 = *reinterpret_cast<const u32x2 *>(&Braw[0][brow[j] + 8]);
        hdr[j] = u32x4{h01.x, h01.y, h23.x, h23.y};
        chunk_scales<0>(hdr[j], dsc[j][0], ndmm[j][0], dsc[j][1], ndmm[j][1]);
        const u32x2 raw = *reinterpret_cast<const u32x2 *>(&Braw[0][brow[j] + 16 + lk]);
        bf[0][j] = dequant8<false>(raw.x, raw.y, dsc[j][0], ndmm[j][0]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) af[0][i] = *reinterpret_cast<const half8 *>(&As[0][afrag + i * 32 * kLdsRow]);

    for (int blk = 0; blk < g.nb; ++blk) {
        const int bb = blk & 1;
        const uint8_t *bcur = Braw[bb];
        const uint8_t *bnext = Braw[bb ^ 1];
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
            const int kc = 4 * blk + c4;
            const int ab = c4 & 1;  // chunk kc's A buffer (4 blk is even)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const int p = ks & 1;
                // operands of the next step: (chunk kc, step ks + 1) or (chunk kc + 1, step 0)
                const int abn = ks < 3 ? ab : ab ^ 1;
                const uint8_t *bsrc = (ks < 3 || c4 < 3) ? bcur : bnext;
                const int kbyte = ks < 3 ? 32 * c4 + (((ks + 1) * 16 + lk) & 31) : 32 * ((c4 + 1) & 3) + lk;
                const int acol = ks < 3 ? (ks + 1) * 16 : 0;
                u32x2 rawn[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    if (ks == 3 && c4 == 3) {
                        const u32x2 h01 = *reinterpret_cast<const u32x2 *>(&bnext[brow[j]]);
                        const u32x2 h23 = *reinterpret_cast<const u32x2 *>(&bnext[brow[j] + 8]);
                        hdr[j] = u32x4{h01.x, h01.y, h23.x, h23.y};
                    }
                    rawn[j] = *reinterpret_cast<const u32x2 *>(&bsrc[brow[j] + 16 + kbyte]);
                }
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    af[p ^ 1][i] = *reinterpret_cast<const half8 *>(&As[abn][afrag + i * 32 * kLdsRow + acol]);
                if (ks == 0) {
                    // A chunk kc + 1 (and B block blk + 1) to the free buffers, then the next loads
                    DOE_PIPE_STORE_A(ab ^ 1);
                    if (c4 == 0) {
                        DOE_PIPE_STORE_B(bb ^ 1);
                        DOE_PIPE_LOAD_B(min(blk + 2, g.nb - 1));
                    }
                    DOE_PIPE_LOAD_A(min(kc + 2, g.nchunk - 1));
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[p][i], bf[p][j], acc[i][j], 0, 0, 0);
                // first half: the B reads, then one LDS read (or write) per MFMA
                if (ks == 3 && c4 == 3) __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
                else __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    if (ks == 0) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
                }
                if (ks == 2) {
                    // every wave's writes of chunk kc + 1 (and block blk + 1) are done, and its
                    // reads of chunk kc's buffers issued: the next chunk may read / overwrite them
                    __builtin_amdgcn_sched_barrier(0);
                    lds_barrier();
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 4; i < 8; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[p][i], bf[p][j], acc[i][j], 0, 0, 0);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    if (ks == 0) {
                        bf[p ^ 1][j] = dequant8<false>(rawn[j].x, rawn[j].y, dsc[j][0], ndmm[j][0]);
                    } else if (ks < 3) {
                        bf[p ^ 1][j] = dequant8<true>(rawn[j].x, rawn[j].y, dsc[j][1], ndmm[j][1]);
                    } else {
                        switch (c4) {  // scales of the next chunk
                            case 0: chunk_scales<1>(hdr[j], dsc[j][0], ndmm[j][0], dsc[j][1], ndmm[j][1]); break;
                            case 1: chunk_scales<2>(hdr[j], dsc[j][0], ndmm[j][0], dsc[j][1], ndmm[j][1]); break;
                            case 2: chunk_scales<3>(hdr[j], dsc[j][0], ndmm[j][0], dsc[j][1], ndmm[j][1]); break;
                            default: chunk_scales<0>(hdr[j], dsc[j][0], ndmm[j][0], dsc[j][1], ndmm[j][1]); break;
                        }
                        bf[p ^ 1][j] = dequant8<false>(rawn[j].x, rawn[j].y, dsc[j][0], ndmm[j][0]);
                    }
                }
                // second half: global loads and the dequant VALU between the MFMAs
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if (ks == 0) {
                        __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);
                        __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
                    }
                    if (ks == 3) __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
                    else __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
#undef DOE_PIPE_LOAD_A
#undef DOE_PIPE_STORE_A
#undef DOE_PIPE_LOAD_B
#undef DOE_PIPE_STORE_B

    // epilogue: D lane l, r: row (r%4) + 8(r/4) + 4(l/32), column l%32
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int ml = i * 32 + (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5);
            const int m = m0 + ml;
            if (m >= g.M) continue;
            const float us = rowscale[ml];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n0 + wave * 64 + j * 32 + lr;
                if (n < g.N) __builtin_nontemporal_store(acc[i][j][r] * us, &g.c[(size_t)m * g.N + n]);
            }
        }
    }
}

// c = sum of the K splits' partial tiles (split order, so the result is
// the same on every run).
// c = the split sum (+ res: the attn_residual / ffn_residual step, c may
// be res), the splits added in order, then the residual.
__global__ __launch_bounds__(256) void sum_splits_kernel(const float *__restrict__ part, float *c, size_t mn,
                                                         int splits, const float *res) {
    const size_t n4 = mn / 4;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        float4 acc = reinterpret_cast<const float4 *>(part)[i];
        for (int s = 1; s < splits; ++s) {
            const float4 v = reinterpret_cast<const float4 *>(part + (size_t)s * mn)[i];
            acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
        }
        if (res) {
            const float4 r = reinterpret_cast<const float4 *>(res)[i];
            acc.x += r.x; acc.y += r.y; acc.z += r.z; acc.w += r.w;
        }
        reinterpret_cast<float4 *>(c)[i] = acc;
    }
    // the last mn % 4 elements
    const size_t i = 4 * n4 + (size_t)blockIdx.x * 256 + threadIdx.x;
    if (blockIdx.x == 0 && i < mn) {
        float acc = part[i];
        for (int s = 1; s < splits; ++s) acc += part[(size_t)s * mn + i];
        if (res) acc += res[i];
        c[i] = acc;
    }
}

// c[row][j] = gelu(gate) * up over the split sums of the gate/up projection
// (the activation step folded in): gate and up columns (2j, 2j + 1) for
// interleaved rows (halves 0) or (j, j + n/2) for [gate | up] (halves 1).
__global__ __launch_bounds__(256) void sum_splits_geglu_kernel(const float *__restrict__ part, float *__restrict__ c,
                                                               int m, int n, int splits, int halves) {
    const int h = n >> 1;
    const size_t mn = (size_t)m * n, total = (size_t)m * h;
    for (size_t o = (size_t)blockIdx.x * 256 + threadIdx.x; o < total; o += (size_t)gridDim.x * 256) {
        const size_t row = o / h, j = o - row * h;
        const size_t gc = row * n + (halves ? j : 2 * j), uc = row * n + (halves ? j + h : 2 * j + 1);
        float g = part[gc], u = part[uc];
        for (int s = 1; s < splits; ++s) {
            g += part[(size_t)s * mn + gc];
            u += part[(size_t)s * mn + uc];
        }
        c[o] = doe_gelu_tanh_clamped(g) * u;
    }
}

// Library-owned workspace (grow-only) for the f16 copy of A and its row scales.
std::mutex g_ws_mu;
void *g_ws = nullptr;
size_t g_ws_bytes = 0;
int g_num_cus = 0;
int g_gemm_f16_operands = 0;  // 1: f32 activations through the f16-operand kernels (one rounding per operand)

// Steps folded around the prompt GEMM (f32 activations only): RMSNorm of
// A's rows in the f16 pre-pass, and a residual add or a GeGLU over gate/up
// column pairs in the pass that sums the K splits.
struct GemmFusion {
    const float *norm_w = nullptr;
    float norm_eps = 0.0f;
    int norm_offset = 0;
    const float *residual = nullptr;  // c += residual (may be c)
    int act = 0;                      // 1: GeGLU over (2j, 2j + 1), 2: over (j, j + n/2); c is [m][n/2]
};

// fmt 0: B Q4_K_M rows; fmt 1: B Q8_0 rows (small-tile kernel only)
int gemm_impl(const void *a, bool a_f32, const void *b_q4k, float *c, int64_t m, int64_t n, int64_t k,
              doe_stream_t stream, int fmt = 0, const GemmFusion &fu = GemmFusion()) {
    const uint16_t *a_bf16 = a_f32 ? nullptr : (const uint16_t *)a;
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(m >= 0 && n >= 0 && k >= 0, DOE_E_INVALID, "negative shape");
    if (m == 0 || n == 0) return DOE_OK;
    DOE_REQUIRE(c, DOE_E_INVALID, "null output");
    hipStream_t st = (hipStream_t)stream;
    const bool epi = fu.residual || fu.act;  // the split-sum pass writes c
    DOE_REQUIRE(a_f32 || (!fu.norm_w && !epi), DOE_E_UNSUPPORTED, "fused steps need f32 activations");
    DOE_REQUIRE(fu.act >= 0 && fu.act <= 2 && !(fu.act && fu.residual), DOE_E_INVALID,
                "activation 0, 1 or 2, and not with a residual");
    DOE_REQUIRE(!fu.act || n % 2 == 0, DOE_E_INVALID, "GeGLU needs an even column count");
    DOE_REQUIRE(!fu.norm_w || (fu.norm_w != c && a != c), DOE_E_INVALID,
                "the norm weight and the activation must not alias the output");
    if (k == 0) {
        // empty reduction: the sum identity (the fused steps need k > 0)
        DOE_REQUIRE(!fu.norm_w && !epi, DOE_E_UNSUPPORTED, "fused steps need k > 0");
        return doe::fill_bytes_async(c, 0, (size_t)m * (size_t)n * sizeof(float), st);
    }
    DOE_REQUIRE(a && b_q4k, DOE_E_INVALID, "null pointer");
    DOE_REQUIRE(((uintptr_t)b_q4k & (fmt ? 3 : 15)) == 0, DOE_E_INVALID, "weight must be %d-byte aligned",
                fmt ? 4 : 16);
    DOE_REQUIRE(!fmt || (uint64_t)n * (uint64_t)((k + 31) / 32) * 34u < (1ull << 31), DOE_E_UNSUPPORTED,
                "Q8_0 weight of %lld rows x %lld columns exceeds 2 GiB", (long long)n, (long long)k);
    DOE_REQUIRE(m <= (1 << 24) && n <= (1 << 24) && k <= (1 << 20) && m * n <= ((int64_t)1 << 40),
                DOE_E_UNSUPPORTED, "q4k_gemm shape too large (m=%lld n=%lld k=%lld)", (long long)m,
                (long long)n, (long long)k);
    // f32 activations run the f32-accurate 128 x 128 kernel (both operands as
    // f16 hi + lo pairs) unless tuned to the f16-operand form; bf16 ones (8
    // significant bits, exact in f16) take 256 x 256 tiles once there are
    // enough of them to fill the CUs, else 128 x 128
    const bool exact = a_f32 && g_gemm_f16_operands == 0;
    const bool big = !exact && fmt == 0 && m >= 256 && n >= 256 && ((m + 255) / 256) * ((n + 255) / 256) >= 256;
    // the large-tile kernel streams whole Q4_K blocks: A padded to 256 nb columns
    const int64_t kp = big ? (k + 255) / 256 * 256 : (k + kBK - 1) / kBK * kBK;
    const size_t a16_bytes = (size_t)m * (size_t)kp * 2 * (exact ? 2 : 1);  // (+ the remainders)
    if (g_num_cus == 0) {
        int dev = 0, cus = 0;
        DOE_HIP_CHECK(hipGetDevice(&dev));
        DOE_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        g_num_cus = cus > 0 ? cus : 256;
    }
    // Short prompts (few 128 x 128 tiles): K split over the grid so that
    // tiles x splits fill the two workgroups per CU that are resident at once
    // (74 KB of LDS each) without spilling into a second round (144 tiles:
    // 3 splits, 432 workgroups, not 4 and 576), at most 32 splits (their
    // partial tiles are written and summed once more; a 128-token prompt
    // measured 4.61, 4.50 and 4.43 ms with at most 8, 16 and 32), each at
    // least one Q4_K block of K.
    // (the f32-accurate kernel: 32-element chunks)
    const int64_t chunk_k = exact ? kXBK : kBK, resident = 2;
    const int64_t nchunk = kp / chunk_k;
    const int64_t small_tiles = ((m + 127) / 128) * ((n + 127) / 128);
    int64_t splits = 1;
    if (!big && small_tiles < resident * g_num_cus) {
        splits = (resident * g_num_cus) / small_tiles;
        if (splits > 32) splits = 32;
        if (splits > nchunk / (256 / chunk_k)) splits = nchunk / (256 / chunk_k);
        if (splits < 1) splits = 1;
    }
    const int64_t kps = (nchunk + splits - 1) / splits;
    splits = (nchunk + kps - 1) / kps;
    const size_t part_off = (a16_bytes + (size_t)m * 4 + 255) & ~(size_t)255;
    const bool use_part = splits > 1 || epi;  // the GEMM writes partial tiles, a second pass writes c
    const size_t need = use_part ? part_off + (size_t)splits * m * n * 4 : a16_bytes + (size_t)m * 4;
    void *ws;
    {
        std::lock_guard<std::mutex> lk(g_ws_mu);
        if (g_ws_bytes < need) {
            doe::retire_workspace(g_ws);  // queued kernels and captured graphs may still use it
            g_ws = nullptr;
            g_ws_bytes = 0;
            DOE_HIP_CHECK(hipMalloc(&g_ws, need));
            g_ws_bytes = need;
        }
        ws = g_ws;
    }
    _Float16 *a16 = (_Float16 *)ws;
    _Float16 *a16lo = exact ? a16 + (size_t)m * (size_t)kp : nullptr;
    int *sig = (int *)((char *)ws + a16_bytes);
    if (a_f32)
        launch_a_rows_f32((const float *)a, fu.norm_w, fu.norm_eps, fu.norm_offset, a16, a16lo, sig, m, k, kp, st);
    else
        hipLaunchKernelGGL(a_rows_to_f16_kernel, dim3((unsigned)m), dim3(256), 0, st, a_bf16, a16, sig, (int)k,
                           (int)kp);
    DOE_LAUNCH_CHECK("a_rows_to_f16_kernel");
    GemmArgs g;
    g.a16 = a16;
    g.a16lo = a16lo;
    g.sig = sig;
    g.b = (const uint8_t *)b_q4k;
    float *part = use_part ? (float *)((char *)ws + part_off) : nullptr;
    g.c = use_part && splits == 1 ? part : c;  // one split: the tile goes to the workspace for the second pass
    g.M = (int)m;
    g.N = (int)n;
    g.Kp = (int)kp;
    g.nb = (int)(fmt ? (k + 31) / 32 : (k + 255) / 256);
    g.nchunk = (int)nchunk;
    g.kps = (int)kps;
    g.part = splits > 1 ? part : nullptr;
    const int bm = big ? 256 : 128, bn = big ? 256 : 128;
    g.tiles_m = (int)((m + bm - 1) / bm);
    g.tiles_n = (int)((n + bn - 1) / bn);
    const int64_t tiles = (int64_t)g.tiles_m * g.tiles_n;
    DOE_REQUIRE(tiles <= 0x7fffffff, DOE_E_UNSUPPORTED, "too many tiles");
    if (big)
        hipLaunchKernelGGL(q4k_gemm_pipe_kernel, dim3((unsigned)tiles), dim3(256), 0, st, g);
    else if (exact && fmt)
        hipLaunchKernelGGL(quant_gemm_exact_kernel<1>, dim3((unsigned)tiles, (unsigned)splits), dim3(256), 0, st, g);
    else if (exact)
        hipLaunchKernelGGL(quant_gemm_exact_kernel<0>, dim3((unsigned)tiles, (unsigned)splits), dim3(256), 0, st, g);
    else if (fmt)
        hipLaunchKernelGGL((quant_gemm_kernel<2, 2, 1>), dim3((unsigned)tiles, (unsigned)splits), dim3(256), 0, st, g);
    else
        hipLaunchKernelGGL((quant_gemm_kernel<2, 2, 0>), dim3((unsigned)tiles, (unsigned)splits), dim3(256), 0, st, g);
    DOE_LAUNCH_CHECK("quant_gemm_kernel");
    if (use_part && fu.act) {
        const size_t total = (size_t)m * (size_t)(n / 2);
        size_t blocks = (total + 255) / 256;
        blocks = blocks < 1 ? 1 : (blocks > 4096 ? 4096 : blocks);
        hipLaunchKernelGGL(sum_splits_geglu_kernel, dim3((unsigned)blocks), dim3(256), 0, st, part, c, (int)m, (int)n,
                           (int)splits, fu.act == 2 ? 1 : 0);
        DOE_LAUNCH_CHECK("sum_splits_geglu_kernel");
    } else if (use_part) {
        const size_t mn = (size_t)m * (size_t)n;
        size_t blocks = (mn / 4 + 255) / 256;
        blocks = blocks < 1 ? 1 : (blocks > 4096 ? 4096 : blocks);
        hipLaunchKernelGGL(sum_splits_kernel, dim3((unsigned)blocks), dim3(256), 0, st, part, c, mn, (int)splits,
                           fu.residual);
        DOE_LAUNCH_CHECK("sum_splits_kernel");
    }
    return DOE_OK;
}

}  // namespace

extern "C" {

}  // extern "C"

namespace doe {
int gemm_set_f16_operands(int v) {
    DOE_REQUIRE(v == 0 || v == 1, DOE_E_INVALID, "quant_gemm.f16_operands is 0 or 1");
    g_gemm_f16_operands = v;
    return DOE_OK;
}
}  // namespace doe

extern "C" {

int doe_q4k_gemm(const uint16_t *a_bf16, const void *b_q4k, float *c, int64_t m, int64_t n,
                 int64_t k, doe_stream_t stream) {
    return gemm_impl(a_bf16, false, b_q4k, c, m, n, k, stream);
}

int doe_q4k_gemm_f32(const float *a, const void *b_q4k, float *c, int64_t m, int64_t n, int64_t k,
                     doe_stream_t stream) {
    return gemm_impl(a, true, b_q4k, c, m, n, k, stream);
}

int doe_q8_0_gemm_f32(const float *a, const void *b_q8_0, float *c, int64_t m, int64_t n, int64_t k,
                      doe_stream_t stream) {
    return gemm_impl(a, true, b_q8_0, c, m, n, k, stream, 1);
}

int doe_quant_gemm_f32_fused(const float *a, const void *b, float *c, int64_t m, int64_t n, int64_t k,
                             int weight_format, const float *norm_weight, float norm_eps, int norm_weight_offset,
                             const float *residual, int activation, doe_stream_t stream) {
    DOE_REQUIRE(weight_format == 0 || weight_format == 1, DOE_E_INVALID, "weight_format is 0 (Q4_K) or 1 (Q8_0)");
    GemmFusion fu;
    fu.norm_w = norm_weight;
    fu.norm_eps = norm_eps;
    fu.norm_offset = norm_weight_offset;
    fu.residual = residual;
    fu.act = activation;
    return gemm_impl(a, true, b, c, m, n, k, stream, weight_format, fu);
}

}  // extern "C"
