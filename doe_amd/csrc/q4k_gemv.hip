// q4k_gemv.hip -- Q4_K_M dequant and decode GEMV (M = 1) for gfx950.
//
// Weight layout (bench/tools/doppler_rdrr_q4k.py:11-15, 56-101, 128-156): row r
// of W[n][k] is ceil(k/256) blocks of 144 bytes; block bytes [0:2] f16 d,
// [2:4] f16 dmin, [4:16] packed 6-bit scales/mins, [16:144] nibbles.  Nibble
// byte 16 + 32c + i holds element 64c + i (sub-block 2c) in its low nibble
// and element 64c + 32 + i (sub-block 2c + 1) in its high nibble.
//
// GEMV work decomposition (one workgroup = `rowslots * R` rows):
//   * a "chunk" is the 32 nibble bytes c of one block: 64 weights from two
//     sub-blocks.  A row has nchunk = ceil(k/64) chunks.
//   * thread t owns chunk t % nchunk of rows slot + r*rowslots (slot =
//     t / nchunk, r < R).  Its 64 activation values never change, so they are
//     staged once per workgroup into LDS as f16 and then held in VGPRs.
//     Consecutive lanes read consecutive 16-byte pieces of one row: the
//     weight stream is fully coalesced with dwordx4 loads.
//   * nibbles become f16 operands with one AND each: a nibble q in the low
//     bits of a half is the subnormal q * 2^-24, a nibble in bits 4..7 is
//     q * 2^-20.  v_dot2_f32_f16 multiplies two such pairs with two activation
//     halves and accumulates in f32; every product is exact.
//   * activations are scaled by a power of two so max|x| sits near 2^14 and
//     split into x_hi = f16(x) and x_lo = f16(x - x_hi): the dot products
//     then carry ~22 bits of the f32 activation.
//   * per sub-block: y += d*sc * sum(q*x) - dmin*m * sum(x).  sum(x) over each
//     sub-block is computed once per workgroup from the f32 activations.
//   * per-chunk partials are reduced through LDS, eight lanes per row.
#include "common.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int kLdsChunkDwords = 36;  // 64 halves + 16 bytes pad: conflict-free b128 reads

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, a), __builtin_bit_cast(half2v, b), c,
                                  false);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (weights are read exactly once).
__device__ __forceinline__ u32x4 load_stream16(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

__device__ __forceinline__ uint32_t pack_half2(_Float16 lo, _Float16 hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, lo) |
           ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

// DPP lane exchanges inside 16-lane rows (no LDS round trip): quad_perm
// [1,0,3,2] and [2,3,0,1] exchange with lane ^ 1 and ^ 2, row_half_mirror
// with lane 7 - i of each 8-lane half, row_mirror with lane 15 - i.  After
// the first three, every lane of an 8-lane group holds the group's sum / max;
// row_mirror then pairs the two groups of a row.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float sum8(float v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    return v + dpp<kDppHalfMirror>(v);
}

__device__ __forceinline__ float sum16(float v) {
    v = sum8(v);
    return v + dpp<kDppMirror>(v);
}

// Scale/min pair of sub-blocks 2*c4 and 2*c4+1 (doppler_rdrr_q4k.py:56-76),
// returned as two bytes each: low byte sub-block 2*c4, high byte 2*c4+1.
__device__ __forceinline__ void q4k_scale_min_pair(uint32_t s0, uint32_t s1, uint32_t s2, int c4,
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
// Dequant: out[r][k] = RN_f32(d*sc*q - dmin*m).  d*sc and dmin*m are exact in
// f32 (11 x 6 significant bits), so one fma rounds the exact value once.
// ---------------------------------------------------------------------------
__global__ void q4k_dequant_kernel(const uint8_t *__restrict__ w, float *__restrict__ out,
                                   int64_t n, int64_t k, int64_t nb) {
    const int64_t total = n * nb * 128;
    for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < total;
         g += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = g / (nb * 128);
        const int64_t rem = g - row * nb * 128;
        const int64_t blk = rem >> 7;
        const int byte = (int)(rem & 127);
        const int c4 = byte >> 5, i = byte & 31;
        const uint8_t *b = w + (row * nb + blk) * DOE_Q4K_BLOCK_BYTES;
        const uint32_t *bw = reinterpret_cast<const uint32_t *>(b);
        const uint32_t h = bw[0];
        uint32_t scp, mnp;
        q4k_scale_min_pair(bw[1], bw[2], bw[3], c4, scp, mnp);
        const float d = doe_half_bits_to_float(h), dmin = doe_half_bits_to_float(h >> 16);
        const uint32_t packed = b[16 + byte];
        const float dsc_lo = d * (float)(scp & 0xffu), dm_lo = dmin * (float)(mnp & 0xffu);
        const float dsc_hi = d * (float)(scp >> 8), dm_hi = dmin * (float)(mnp >> 8);
        const int64_t lo = blk * 256 + c4 * 64 + i, hi = lo + 32;
        if (lo < k) out[row * k + lo] = fmaf(dsc_lo, (float)(packed & 15u), -dm_lo);
        if (hi < k) out[row * k + hi] = fmaf(dsc_hi, (float)(packed >> 4), -dm_hi);
    }
}

// ---------------------------------------------------------------------------
// GEMV.
// LDS layout (dynamic): xh[nchunk*36] dwords, xl[nchunk*36] dwords (f16 pairs
// of x_hi / x_lo), sx[2*nchunk] f32 sub-block sums, sig[nchunk] i32 chunk
// scale exponents, red[rows_wg*nchunk] f32 partials.
// Within a chunk, dwords 0..15 hold the low sub-block and 16..31 the high one;
// each 4-element group (e0,e1,e2,e3) is stored as pairs (e0,e2), (e1,e3) so
// that `D & 0x000F000F` (bytes 0 and 2 of a nibble dword) meets (e0,e2) and
// `(D >> 8) & 0x000F000F` meets (e1,e3).
// Each chunk's 64 activations are scaled by their own power of two (max|x|
// of the chunk near 2^14); the chunk's partial is scaled back exactly.
// ---------------------------------------------------------------------------
// Stages activation quad `qd` (elements 4qd..4qd+3): sub-block sum, chunk
// scale exponent, and the scaled x_hi / x_lo halves in dot2 pair order.
__device__ __forceinline__ void stage_quad(int qd, bool valid, const float *v, uint32_t *xh,
                                           uint32_t *xl, float *sx, int *sig) {
    const float s = sum8((v[0] + v[1]) + (v[2] + v[3]));
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = fmaxf(amax, dpp<kDppXor1>(amax));
    amax = fmaxf(amax, dpp<kDppXor2>(amax));
    amax = fmaxf(amax, dpp<kDppHalfMirror>(amax));
    amax = fmaxf(amax, dpp<kDppMirror>(amax));
    int sigma = 0;
    if (amax > 0.0f && amax <= 3.0e38f) {
        sigma = 14 - __builtin_amdgcn_frexp_expf(amax);
        sigma = sigma < -100 ? -100 : (sigma > 100 ? 100 : sigma);
    }
    const float xs = __builtin_amdgcn_ldexpf(1.0f, sigma);
    if (!valid) return;
    if ((qd & 7) == 0) sx[qd >> 3] = s;
    if ((qd & 15) == 0) sig[qd >> 4] = sigma;
    _Float16 hi[4], lo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float t = v[j] * xs;
        hi[j] = (_Float16)t;
        lo[j] = (_Float16)(t - (float)hi[j]);
    }
    const int off = (qd >> 4) * kLdsChunkDwords + 2 * (qd & 15);
    *reinterpret_cast<uint2 *>(xh + off) = make_uint2(pack_half2(hi[0], hi[2]), pack_half2(hi[1], hi[3]));
    *reinterpret_cast<uint2 *>(xl + off) = make_uint2(pack_half2(lo[0], lo[2]), pack_half2(lo[1], lo[3]));
}

// Optional fusions around the GEMV (all off for the plain matmul_q4k op).
struct GemvFusion {
    const float *norm_w;    // RMSNorm weight: x <- x * inv_rms * (w or 1 + w)
    float norm_eps;
    int norm_offset;        // 1: (1 + w) form
    const float *residual;  // y[i] += residual[i]
    int gated;              // rows (2i, 2i+1) -> y[i] = gelu(y_2i) * y_2i+1
    // RoPE + KV-cache write over a fused [q; k; v] projection whose q and k
    // rows come as interleaved rotation pairs (row 2i = dim i, row 2i+1 =
    // dim i + head_dim/2 of the rotate-half form): pairs of q/k rows are
    // rotated by freq_cis[pos][i]; k and v rows are also stored as f16 into
    // the caches [kv_heads][max_seq][head_dim] at pos.
    int rope_kv;
    // Activation = the combine of split-attention partials (o [heads][S][D],
    // ml [heads][S][2] = (m, l) in log2 units): x[h D + d] =
    // sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), M = max_s m_s.
    const float *attn_o;
    const float *attn_ml;
    int attn_splits, attn_head_dim;
    const float *freq_cis;
    const int32_t *pos_dev;
    _Float16 *k_cache, *v_cache;
    int q_rows, kv_rows, head_dim, max_seq;
    // Activation given as x + x_parts[0] + ... + x_parts[x_nparts - 1]
    // (each part k floats, added in that order); workgroup (0, 0) stores the
    // sum to x_sum when non-NULL.  Matrix-core kernel only.
    const float *x_parts;
    int x_nparts;
    float *x_sum;
    // K split into parts: K range s stores its row sums to y_parts[s n + row]
    // with plain stores (no residual, no atomics); the consumer adds them.
    float *y_parts;
    // Residual given as residual + res_parts[0] + ... + res_parts[res_nparts
    // - 1] (each n floats, added in that order): a consumer forms the sum a
    // producer's activation prologue formed, instead of reading it stored.
    // Matrix-core kernel, whole rows or output parts.
    const float *res_parts;
    int res_nparts;
};

constexpr int kMaxXParts = 4;  // activation parts a GEMV adds in its prologue

// Epilogue of one (even row, odd row) pair of a fused q/k/v projection.
__device__ __forceinline__ DoeRopeKv rope_kv_of(const GemvFusion &fz) {
    return DoeRopeKv{fz.freq_cis, fz.pos_dev, fz.k_cache, fz.v_cache, fz.q_rows, fz.kv_rows, fz.head_dim,
                     fz.max_seq};
}
__device__ __forceinline__ void rope_kv_pair(const GemvFusion &fz, int row, float s0, float s1,
                                             float *__restrict__ y) {
    doe_rope_kv_pair(rope_kv_of(fz), row, s0, s1, y);
}

// PRO: activation prologue -- 0 plain f32 load, 1 fused RMSNorm, 2 combine of
// split-attention partials (S <= kAttnMaxSplits).
constexpr int kAttnMaxSplits = 8;

template <int R, int Q, int PRO>
__global__ __launch_bounds__(1024) void q4k_gemv_kernel(const uint8_t *__restrict__ w,
                                                        const float *__restrict__ x,
                                                        float *__restrict__ y, int n, int k, int nb,
                                                        int nchunk, int rowslots, GemvFusion fz) {
    extern __shared__ uint32_t smem[];
    uint32_t *xh = smem;
    uint32_t *xl = xh + nchunk * kLdsChunkDwords;
    float *sx = reinterpret_cast<float *>(xl + nchunk * kLdsChunkDwords);
    int *sig = reinterpret_cast<int *>(sx + 2 * nchunk);
    float *red = reinterpret_cast<float *>(sig + nchunk);
    const int rows_wg = rowslots * R;
    float *wsum = red + rows_wg * nchunk;  // [16] per-wave partial sums (RMSNorm)

    const int tid = threadIdx.x;
    const int nthreads = blockDim.x;
    const int nquads = nchunk * 16;
    const int active = rowslots * nchunk;
    const bool worker = tid < active;
    const int chunk = worker ? tid % nchunk : 0;
    const int slot = worker ? tid / nchunk : 0;
    const int blk = chunk >> 2, c4 = chunk & 3;
    const int row0 = blockIdx.x * rows_wg + slot;

    // Phase 1: this thread's activation quads go out first (vector-memory
    // returns are in order, so staging never waits on the weight stream),
    // then its weight bytes.  Each thread stages Q quads in registers; the
    // host picks Q >= nquads / nthreads when it can.
    // Loads are unconditional (indices clamped into range, results masked
    // later) so they stay in straight-line code and the compiler can wait on
    // the activation without waiting on the weights.
    constexpr bool NORM = PRO == 1, ATTN = PRO == 2;
    float xv[Q][4];
    float4 ao[ATTN ? Q : 1][ATTN ? kAttnMaxSplits : 1];
    float2 aml[ATTN ? Q : 1][ATTN ? kAttnMaxSplits : 1];
    if (ATTN) {
        // the partials of this thread's quads (a quad never straddles heads)
        const int S = fz.attn_splits, D = fz.attn_head_dim;
#pragma unroll
        for (int it = 0; it < Q; ++it) {
            const int e = min((tid + it * nthreads) * 4, k - 4);
            const int h = e / D, d = e - h * D;
#pragma unroll
            for (int sp = 0; sp < kAttnMaxSplits; ++sp) {
                const int ss = min(sp, S - 1);
                ao[it][sp] = *reinterpret_cast<const float4 *>(fz.attn_o + ((size_t)h * S + ss) * D + d);
                aml[it][sp] = *reinterpret_cast<const float2 *>(fz.attn_ml + ((size_t)h * S + ss) * 2);
            }
        }
    } else {
#pragma unroll
        for (int it = 0; it < Q; ++it) {
            const int e = (tid + it * nthreads) * 4;
#pragma unroll
            for (int j = 0; j < 4; ++j) xv[it][j] = x[min(e + j, k - 1)];  // masked when staged
        }
    }
    float nwv[NORM ? Q : 1][4];
    if (NORM) {
#pragma unroll
        for (int it = 0; it < Q; ++it) {
            const int e = (tid + it * nthreads) * 4;
#pragma unroll
            for (int j = 0; j < 4; ++j) nwv[it][j] = fz.norm_w[min(e + j, k - 1)];
        }
    }
    // keep the activation loads ahead of the weight loads in issue order
    __builtin_amdgcn_sched_barrier(0);
    // (one 16-byte header load per chunk thread measured faster than one
    // dword per thread shared across the block's lane quad by DPP, and than
    // reading the workgroup's rows as consecutive granules through LDS)
    u32x4 hdr[R], qa[R], qb[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r * rowslots, n - 1);
        const uint8_t *p = w + ((size_t)row * nb + blk) * DOE_Q4K_BLOCK_BYTES;
        hdr[r] = load_stream16(p);
        qa[r] = load_stream16(p + 16 + 32 * c4);
        qb[r] = load_stream16(p + 32 + 32 * c4);
    }
    __builtin_amdgcn_sched_barrier(0);

    if (ATTN) {
        const int S = fz.attn_splits;
#pragma unroll
        for (int it = 0; it < Q; ++it) {
            float M = -INFINITY;
#pragma unroll
            for (int sp = 0; sp < kAttnMaxSplits; ++sp)
                if (sp < S) M = fmaxf(M, aml[it][sp].x);
            float L = 0.0f, O0 = 0.0f, O1 = 0.0f, O2 = 0.0f, O3 = 0.0f;
            if (M != -INFINITY) {
#pragma unroll
                for (int sp = 0; sp < kAttnMaxSplits; ++sp) {
                    if (sp < S) {
                        const float f = exp2f(aml[it][sp].x - M);
                        L = fmaf(aml[it][sp].y, f, L);
                        O0 = fmaf(ao[it][sp].x, f, O0);
                        O1 = fmaf(ao[it][sp].y, f, O1);
                        O2 = fmaf(ao[it][sp].z, f, O2);
                        O3 = fmaf(ao[it][sp].w, f, O3);
                    }
                }
            }
            const float r = L > 0.0f ? 1.0f / L : 0.0f;
            xv[it][0] = O0 * r;
            xv[it][1] = O1 * r;
            xv[it][2] = O2 * r;
            xv[it][3] = O3 * r;
        }
    }

    // Fused RMSNorm (the host guarantees Q * nthreads >= nquads): stage
    // x * (w or 1 + w) and multiply each row sum by 1 / sqrt(mean(x^2) + eps)
    // at the end -- the same product, so the sum of squares is reduced in
    // the shadow of the staging instead of behind a barrier of its own.
    // Each wave leaves its share in wsum before the staging barrier.
    if (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int it = 0; it < Q; ++it) {
            const int e = (tid + it * nthreads) * 4;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float v = (e + j < k) ? xv[it][j] : 0.0f;
                ss = fmaf(v, v, ss);
                const float nw = nwv[it][j];
                xv[it][j] *= fz.norm_offset ? 1.0f + nw : nw;
            }
        }
        ss = sum16(ss);  // every lane of a 16-lane row holds its row's sum
        const float wsum_wave = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 0)) +
                                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 16)) +
                                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 32)) +
                                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 48));
        if ((tid & 63) == 0) wsum[tid >> 6] = wsum_wave;
    }

    // Phase 2: stage the activation once per workgroup.  The 16 quads of a
    // chunk are 16 consecutive lanes and the 8 quads of a sub-block 8 lanes
    // (nthreads % 64 == 0, nquads % 16 == 0), so every shuffle group below
    // is either fully active or fully idle.
#pragma unroll
    for (int it = 0; it < Q; ++it) {
        const int qd = tid + it * nthreads;
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (qd * 4 + j < k) ? xv[it][j] : 0.0f;
        stage_quad(qd, qd < nquads, v, xh, xl, sx, sig);
    }
    for (int qd = tid + Q * nthreads; qd < nquads; qd += nthreads) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (qd * 4 + j < k) ? x[qd * 4 + j] : 0.0f;
        stage_quad(qd, true, v, xh, xl, sx, sig);
    }
    __syncthreads();

    // Phase 3: dot products of this thread's chunk for its R rows.
    if (worker) {
        uint32_t xhv[32], xlv[32];
        const u32x4 *xh4 = reinterpret_cast<const u32x4 *>(xh + chunk * kLdsChunkDwords);
        const u32x4 *xl4 = reinterpret_cast<const u32x4 *>(xl + chunk * kLdsChunkDwords);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const u32x4 a = xh4[i], b = xl4[i];
            xhv[4 * i] = a.x; xhv[4 * i + 1] = a.y; xhv[4 * i + 2] = a.z; xhv[4 * i + 3] = a.w;
            xlv[4 * i] = b.x; xlv[4 * i + 1] = b.y; xlv[4 * i + 2] = b.z; xlv[4 * i + 3] = b.w;
        }
        const float sxl = sx[2 * chunk], sxh = sx[2 * chunk + 1];
        const int sigma = sig[chunk];
        const float f_lo = __builtin_amdgcn_ldexpf(1.0f, 24 - sigma);
        const float f_hi = __builtin_amdgcn_ldexpf(1.0f, 20 - sigma);

#pragma unroll
        for (int r = 0; r < R; ++r) {
            uint32_t scp, mnp;
            q4k_scale_min_pair(hdr[r].y, hdr[r].z, hdr[r].w, c4, scp, mnp);
            const float d = doe_half_bits_to_float(hdr[r].x);
            const float dmin = doe_half_bits_to_float(hdr[r].x >> 16);
            const uint32_t q[8] = {qa[r].x, qa[r].y, qa[r].z, qa[r].w,
                                   qb[r].x, qb[r].y, qb[r].z, qb[r].w};
            float lo_a = 0.0f, lo_b = 0.0f, hi_a = 0.0f, hi_b = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t dw = q[i], ew = dw >> 8;
                const uint32_t p0 = dw & 0x000f000fu, p1 = ew & 0x000f000fu;
                const uint32_t p2 = dw & 0x00f000f0u, p3 = ew & 0x00f000f0u;
                lo_a = dot2(p0, xhv[2 * i], lo_a);
                lo_a = dot2(p1, xhv[2 * i + 1], lo_a);
                hi_a = dot2(p2, xhv[16 + 2 * i], hi_a);
                hi_a = dot2(p3, xhv[16 + 2 * i + 1], hi_a);
                lo_b = dot2(p0, xlv[2 * i], lo_b);
                lo_b = dot2(p1, xlv[2 * i + 1], lo_b);
                hi_b = dot2(p2, xlv[16 + 2 * i], hi_b);
                hi_b = dot2(p3, xlv[16 + 2 * i + 1], hi_b);
            }
            const float qx_lo = (lo_a + lo_b) * f_lo;
            const float qx_hi = (hi_a + hi_b) * f_hi;
            const float sc_lo = (float)(scp & 0xffu), sc_hi = (float)(scp >> 8);
            const float m_lo = (float)(mnp & 0xffu), m_hi = (float)(mnp >> 8);
            const float part = d * (sc_lo * qx_lo + sc_hi * qx_hi) - dmin * (m_lo * sxl + m_hi * sxh);
            red[(slot + r * rowslots) * nchunk + chunk] = part;
        }
    }
    __syncthreads();

    // Phase 4: reduce each row's nchunk partials, eight lanes per row.
    float inv_rms = 1.0f;
    if (NORM) {
        float tot = 0.0f;
        for (int i = 0; i < (nthreads >> 6); ++i) tot += wsum[i];
        inv_rms = 1.0f / sqrtf(tot / (float)k + fz.norm_eps);
    }
    for (int idx = tid; idx < rows_wg * 8; idx += nthreads) {
        const int lr = idx >> 3, l8 = idx & 7;
        float s = 0.0f;
        for (int j = l8; j < nchunk; j += 8) s += red[lr * nchunk + j];
        s = sum8(s);
        if (NORM) s *= inv_rms;
        const int row = blockIdx.x * rows_wg + lr;
        if (fz.gated) {
            // the partner row (lr ^ 1) is the other 8-lane group of this row of 16 lanes
            const float other = dpp<kDppMirror>(s);
            if (l8 == 0 && (lr & 1) == 0 && row < n) y[row >> 1] = doe_gelu_tanh_clamped(s) * other;
        } else if (fz.rope_kv) {
            const float other = dpp<kDppMirror>(s);
            if (l8 == 0 && (lr & 1) == 0 && row < n) rope_kv_pair(fz, row, s, other, y);
        } else if (l8 == 0 && row < n) {
            y[row] = fz.residual ? s + fz.residual[row] : s;
        }
    }
}

// ---------------------------------------------------------------------------
// GEMV on the matrix cores (k <= 16 blocks).  One workgroup owns 16 rows; wave
// b owns Q4_K block b of those rows and is self-contained up to the final
// cross-block row sum:
//   * it reads the 16 rows' 144-byte block b as consecutive 16-byte granules
//     (lane q -> row q / 9, piece q % 9) and regroups them through its own
//     LDS slice;
//   * it stages its own 256 activations (lane 16 g + i holds elements
//     64 g + 4 i .. +3, i.e. chunk g of the block) into an "A image";
//   * eight v_mfma_f32_16x16x32_f16 compute D[variant][row] with B = nibbles
//     as f16 subnormals (q * 2^-24 low, q * 2^-20 high, exact products) and
//     A = the 16 variants (sub-block 2g + s, x_hi or x_lo) of the staged
//     activations.  MFMA step j feeds lane group g's nibble dword j (bytes
//     4j..4j+3 of chunk g: elements 4j..4j+3 of sub-blocks 2g and 2g + 1);
//     variant m = 4g + 2s + h is nonzero only for lane group g's data of
//     sub-block 2g + s, so A is zero except in lanes m / 4 == g;
//   * D lands with lane (g, row) holding variants 4g..4g+3: exactly the four
//     partial sums the per-chunk scale formula (d*sc, dmin*m of sub-blocks
//     2g, 2g + 1) needs, in the lane that also loaded that row's header and
//     staged chunk g's activation sums.
// The A image of step j is [chunk g][part h][type s] 16-byte slots with the
// two non-matching halves zero ({pair0, pair1, 0, 0} for s = 0, {0, 0, pair0,
// pair1} for s = 1), followed by a zero slot that all inactive lanes read.
// ---------------------------------------------------------------------------
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMfmaMaxBlocks = 64;                 // <= 16 waves of <= 4 blocks each
constexpr int kMfmaRowBytes = 160;                 // LDS bytes per regrouped row block (144 + 16)
constexpr int kMfmaAStep = 68;                     // dwords per MFMA step in the A image (64 + 4 zero)
constexpr int kMfmaAImgDwords = 8 * kMfmaAStep;    // one block's activation image (2176 bytes)

// Activation images per wave: up to three blocks' images are staged ahead.
constexpr int mfma_images(int bpw) { return bpw < 3 ? bpw : 3; }
constexpr int mfma_wave_lds(int bpw) { return 16 * kMfmaRowBytes + mfma_images(bpw) * kMfmaAImgDwords * 4; }

size_t gemv_mfma_lds_bytes(int nwaves, int bpw) {
    return (size_t)nwaves * mfma_wave_lds(bpw) + (size_t)17 * nwaves * 4;
}

// Sum over the four 16-lane rows of a wave (lanes i, i + 16, i + 32, i + 48)
// with the gfx950 cross-row swaps; every lane ends with its column's total.
__device__ __forceinline__ float sum_rows4(float v) {
    auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
    auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
}

// BPW consecutive blocks per wave (BPW = ceil(nb / 16), so a workgroup of at
// most 16 waves covers the row): the weight loads of all of the wave's blocks
// are issued up front in block order and the blocks are then processed one
// after another through the same LDS slice, so the first block's MFMAs run
// while the later blocks' bytes arrive.
// XV: the activation is read as one float4 per lane (x 16-byte aligned and
// k % 4 == 0), else as four clamped dwords.  Both forms are branch-free so the
// activation loads stay ahead of the weight stream.
// EPI: 1 the residual comes with parts (fz.res_parts); 2 the q/k/v epilogue
// with its rotation fetched ahead (the position a scalar load at the start,
// each row pair's cos / sin once the weight loads are out).  Forms of their
// own, so the others keep their register count (61 VGPRs: eight waves per
// SIMD; 65 measured slower).
template <int PRO, int BPW, int XV, int EPI = 0>
__global__ __launch_bounds__(1024) void q4k_gemv_mfma_kernel(const uint8_t *__restrict__ w,
                                                             const float *x,
                                                             float *__restrict__ y, int n, int k,
                                                             int nb, int nbs, GemvFusion fz) {
    constexpr bool NORM = PRO == 1, ATTN = PRO == 2;
    constexpr int NA = mfma_images(BPW), WAVE_LDS = mfma_wave_lds(BPW);
    static_assert(!ATTN || BPW == 1, "the attention-combine prologue is single-block");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    uint8_t *wimg = lds + wave * WAVE_LDS;
    uint32_t *aimg = reinterpret_cast<uint32_t *>(wimg + 16 * kMfmaRowBytes);
    float *red = reinterpret_cast<float *>(lds + nwaves * WAVE_LDS);  // [16][nwaves] row partials
    float *ssq = red + 16 * nwaves;                                       // [nwaves] sums of squares
    // K split: workgroup (x, y) owns blocks [y * nbs, min(nb, (y + 1) * nbs)).
    const int row0 = blockIdx.x * 16, kb1 = min(nb, ((int)blockIdx.y + 1) * nbs);
    const int b0 = (int)blockIdx.y * nbs + wave * BPW;

    // Activation operands first (vector-memory returns are in order, so the
    // staging below never waits on the weight stream).
    float v[BPW][4], nwv[NORM ? BPW : 1][4];
    float4 ao[ATTN ? kAttnMaxSplits : 1];
    float2 aml[ATTN ? kAttnMaxSplits : 1];
    // activation parts (fz.x_parts): up to two blocks per wave
    constexpr int XPB = (!ATTN && BPW <= 2) ? BPW : 0;
    float4 xp[XPB > 0 ? XPB : 1][kMaxXParts];
#pragma unroll
    for (int u = 0; u < BPW; ++u) {
        const int e = (b0 + u) * 256 + lane * 4;  // this lane's four activations of block b0 + u
        if (ATTN) {
            // a lane's four elements lie in one head (head_dim % 4 == 0)
            const int S = fz.attn_splits, D = fz.attn_head_dim;
            const int ec = min(e, k - 4), h = ec / D, d = ec - h * D;
#pragma unroll
            for (int sp = 0; sp < kAttnMaxSplits; ++sp) {
                if (sp < S) {  // S is uniform: only the existing splits are read
                    ao[sp] = *reinterpret_cast<const float4 *>(fz.attn_o + ((size_t)h * S + sp) * D + d);
                    aml[sp] = *reinterpret_cast<const float2 *>(fz.attn_ml + ((size_t)h * S + sp) * 2);
                }
            }
        } else if (XV) {
            const float4 f = *reinterpret_cast<const float4 *>(x + min(e, k - 4));  // masked below
            v[u][0] = f.x; v[u][1] = f.y; v[u][2] = f.z; v[u][3] = f.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[u][j] = x[min(e + j, k - 1)];  // masked below
        }
        if (XPB > 0 && fz.x_nparts > 0) {
            // the activation's parts: loads issued with the activation's,
            // added once the weight loads are out (below)
#pragma unroll
            for (int sp = 0; sp < kMaxXParts; ++sp) {
                if (sp < fz.x_nparts) {
                    const float *pp = fz.x_parts + (size_t)sp * k;
                    float4 &t = xp[XPB > 0 ? u : 0][sp];
                    if (XV) {
                        t = *reinterpret_cast<const float4 *>(pp + min(e, k - 4));
                    } else {
                        t.x = pp[min(e, k - 1)];
                        t.y = pp[min(e + 1, k - 1)];
                        t.z = pp[min(e + 2, k - 1)];
                        t.w = pp[min(e + 3, k - 1)];
                    }
                }
            }
        }
        if (NORM && XV) {  // (XV also covers the norm weight's alignment)
            const float4 f = *reinterpret_cast<const float4 *>(fz.norm_w + min(e, k - 4));
            nwv[NORM ? u : 0][0] = f.x; nwv[NORM ? u : 0][1] = f.y;
            nwv[NORM ? u : 0][2] = f.z; nwv[NORM ? u : 0][3] = f.w;
        } else if (NORM) {
#pragma unroll
            for (int j = 0; j < 4; ++j) nwv[NORM ? u : 0][j] = fz.norm_w[min(e + j, k - 1)];
        }
    }
    // The residual of the epilogue's rows, loaded with the activation so the
    // last store does not wait on a load (K split: range 0 adds it when the
    // ranges go to parts; atomic ranges add into a y that holds it already).
    const bool has_res = fz.residual && blockIdx.y == 0 && (fz.y_parts || gridDim.y == 1);
    // (its parts are loaded here and added once the weight loads are out:
    // an add here would wait for them before the weight loads go out)
    constexpr bool RP = EPI == 1, ROPE = EPI == 2;
    float rres[RP ? 1 + kMaxXParts : 1] = {};
    if (has_res && tid < 16) {
        const int rr = min(row0 + tid, n - 1);
        rres[0] = fz.residual[rr];
        if constexpr (RP) {
#pragma unroll
            for (int sp = 0; sp < kMaxXParts; ++sp)
                if (sp < fz.res_nparts) rres[1 + sp] = fz.res_parts[(size_t)sp * n + rr];
        }
    }
    const int rope_pos = ROPE ? doe_rope_pos_scalar(fz.pos_dev) : 0;
    // (x is not __restrict__: with it its loads count as invariant and were
    // sunk past the weight loads; this memory clobber keeps the order)
    __asm__ volatile("" ::: "memory");
    // Block b of the 16 rows: granule q -> row q / 9, piece q % 9.
    const size_t rowbytes = (size_t)nb * DOE_Q4K_BLOCK_BYTES;
    u32x4 wv[BPW][3];
#pragma unroll
    for (int u = 0; u < BPW; ++u) {
        const int blk = min(b0 + u, kb1 - 1);  // past the range: a valid block, unused
#pragma unroll
        for (int s = 0; s < 3; ++s) {
            const int q = min(lane + 64 * s, 143);
            const int r = min(row0 + q / 9, n - 1);
            wv[u][s] = load_stream16(w + (size_t)r * rowbytes + blk * DOE_Q4K_BLOCK_BYTES + (q % 9) * 16);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // (every lane issues the two rotation loads, from an in-range position,
    // so no path skips them and the waits count the loads exactly)
    float rope_c = 1.0f, rope_s = 0.0f;
    if constexpr (ROPE) {
        const int i = ((row0 + (tid & 15)) % fz.head_dim) >> 1;
        const int p = min(max(rope_pos, 0), fz.max_seq - 1);
        const float *src = fz.freq_cis + ((size_t)p * (fz.head_dim >> 1) + i) * 2;
        rope_c = src[0];
        rope_s = src[1];
    }
    float rpre = rres[0];
    if constexpr (RP) {
#pragma unroll
        for (int sp = 0; sp < kMaxXParts; ++sp)
            if (sp < fz.res_nparts) rpre += rres[1 + sp];
    }

    if (XPB > 0 && fz.x_nparts > 0) {
        // x + part 0 + part 1 + ..., in that order; workgroup (0, 0) keeps
        // the sum (the residual stream the later steps read)
        const bool keep = fz.x_sum && blockIdx.x == 0 && blockIdx.y == 0;
#pragma unroll
        for (int u = 0; u < XPB; ++u) {
#pragma unroll
            for (int sp = 0; sp < kMaxXParts; ++sp) {
                if (sp < fz.x_nparts) {
                    const float4 t = xp[u][sp];
                    v[u][0] += t.x; v[u][1] += t.y; v[u][2] += t.z; v[u][3] += t.w;
                }
            }
            if (keep) {
                const int e = (b0 + u) * 256 + lane * 4;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (e + j < kb1 * 256 && e + j < k)
                        __hip_atomic_store(fz.x_sum + e + j, v[u][j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }

    if (ATTN) {
        const int S = fz.attn_splits;
        float M = -INFINITY;
#pragma unroll
        for (int sp = 0; sp < kAttnMaxSplits; ++sp)
            if (sp < S) M = fmaxf(M, aml[sp].x);
        float L = 0.0f, O0 = 0.0f, O1 = 0.0f, O2 = 0.0f, O3 = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int sp = 0; sp < kAttnMaxSplits; ++sp) {
                if (sp < S) {
                    const float f = exp2f(aml[sp].x - M);
                    L = fmaf(aml[sp].y, f, L);
                    O0 = fmaf(ao[sp].x, f, O0);
                    O1 = fmaf(ao[sp].y, f, O1);
                    O2 = fmaf(ao[sp].z, f, O2);
                    O3 = fmaf(ao[sp].w, f, O3);
                }
            }
        }
        const float rl = L > 0.0f ? 1.0f / L : 0.0f;
        v[0][0] = O0 * rl; v[0][1] = O1 * rl; v[0][2] = O2 * rl; v[0][3] = O3 * rl;
    }
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < BPW; ++u) {
        const int e = (b0 + u) * 256 + lane * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (e + j >= k) v[u][j] = 0.0f;
            if (NORM) {
                // RMSNorm: stage x * (w or 1 + w); the row sums are multiplied
                // by 1 / sqrt(mean(x^2) + eps) at the end (the same product).
                ss = fmaf(v[u][j], v[u][j], ss);
                const float nw = nwv[NORM ? u : 0][j];
                v[u][j] *= fz.norm_offset ? 1.0f + nw : nw;
            }
        }
    }
    if (NORM) {
        ss = sum_rows4(sum16(ss));
        if (lane == 0) ssq[wave] = ss;
    }

    const int g = lane >> 4, i16 = lane & 15, m = lane & 15;
    const int nchunk = (k + 63) >> 6;
    // Stage block b0 + u's activation image into image slot u % NA: lane
    // 16 g + i holds chunk g, quad i (a chunk is one DPP row, a sub-block a
    // half); returns the chunk's scale exponent and sub-block sums.
    float sxl[BPW], sxh[BPW];
    int sgm[BPW];
    auto stage = [&](int u) __attribute__((always_inline)) {
        uint32_t *img = aimg + (u % NA) * kMfmaAImgDwords;
        const float ssum = sum8((v[u][0] + v[u][1]) + (v[u][2] + v[u][3]));
        const float sother = dpp<kDppMirror>(ssum);  // the other sub-block of the chunk
        sxl[u] = i16 < 8 ? ssum : sother;
        sxh[u] = i16 < 8 ? sother : ssum;
        float amax = fmaxf(fmaxf(fabsf(v[u][0]), fabsf(v[u][1])), fmaxf(fabsf(v[u][2]), fabsf(v[u][3])));
        amax = fmaxf(amax, dpp<kDppXor1>(amax));
        amax = fmaxf(amax, dpp<kDppXor2>(amax));
        amax = fmaxf(amax, dpp<kDppHalfMirror>(amax));
        amax = fmaxf(amax, dpp<kDppMirror>(amax));
        int sigma = 0;
        if (amax > 0.0f && amax <= 3.0e38f) {
            sigma = 14 - __builtin_amdgcn_frexp_expf(amax);
            sigma = sigma < -100 ? -100 : (sigma > 100 ? 100 : sigma);
        }
        sgm[u] = sigma;
        const float xs = __builtin_amdgcn_ldexpf(1.0f, sigma);
        _Float16 hi[4], lo[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float t = v[u][j] * xs;
            hi[j] = (_Float16)t;
            lo[j] = (_Float16)(t - (float)hi[j]);
        }
        const int s = i16 >> 3, jj = i16 & 7;
        const uint32_t h0 = pack_half2(hi[0], hi[2]), h1 = pack_half2(hi[1], hi[3]);
        const uint32_t l0 = pack_half2(lo[0], lo[2]), l1 = pack_half2(lo[1], lo[3]);
        uint32_t *dst = img + jj * kMfmaAStep + g * 16 + s * 4;
        *reinterpret_cast<u32x4 *>(dst) = s ? u32x4{0, 0, h0, h1} : u32x4{h0, h1, 0, 0};
        *reinterpret_cast<u32x4 *>(dst + 8) = s ? u32x4{0, 0, l0, l1} : u32x4{l0, l1, 0, 0};
        if (u < NA && lane < 8) *reinterpret_cast<u32x4 *>(img + lane * kMfmaAStep + 64) = u32x4{0, 0, 0, 0};
    };
    // The first NA blocks' images are staged while the weights are in flight.
#pragma unroll
    for (int u = 0; u < NA; ++u)
        if (b0 + u < kb1) stage(u);
    // LDS operations of one wave complete in order (an image is read before a
    // later block overwrites it); the wave barriers keep the compiler from
    // moving reads above writes.
    __builtin_amdgcn_wave_barrier();
    float part = 0.0f;
    u32x4 areg[8];
    auto read_a = [&](int u) __attribute__((always_inline)) {
        const int c = 4 * (b0 + u) + g;
        const bool act = (m >> 2) == g && c < nchunk;
        const uint32_t *img = aimg + (u % NA) * kMfmaAImgDwords;
        const int abase = act ? g * 16 + (m & 1) * 8 + ((m >> 1) & 1) * 4 : 64;
#pragma unroll
        for (int j = 0; j < 8; ++j) areg[j] = *reinterpret_cast<const u32x4 *>(img + j * kMfmaAStep + abase);
    };
    read_a(0);  // before the weights arrive
#pragma unroll
    for (int u = 0; u < BPW; ++u) {
        const int b = b0 + u;
        if (b >= kb1) break;  // wave-uniform
        if (u >= NA) {
            stage(u);  // slot u % NA: block u - NA is done with it
            __builtin_amdgcn_wave_barrier();
        }
#pragma unroll
        for (int s = 0; s < 3; ++s) {
            const int q = lane + 64 * s;
            if (q < 144) *reinterpret_cast<u32x4 *>(wimg + (q / 9) * kMfmaRowBytes + (q % 9) * 16) = wv[u][s];
        }
        __builtin_amdgcn_wave_barrier();
        if (u > 0) read_a(u);
        const uint8_t *rp = wimg + i16 * kMfmaRowBytes;  // lane (g, row i16)
        const u32x4 hdr = *reinterpret_cast<const u32x4 *>(rp);
        const u32x4 qa = *reinterpret_cast<const u32x4 *>(rp + 16 + 32 * g);
        const u32x4 qb = *reinterpret_cast<const u32x4 *>(rp + 32 + 32 * g);
        f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t dw = j < 4 ? qa[j] : qb[j - 4], ew = dw >> 8;
            const u32x4 bw = {dw & 0x000f000fu, ew & 0x000f000fu, dw & 0x00f000f0u, ew & 0x00f000f0u};
            acc[j & 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, areg[j]),
                                                                __builtin_bit_cast(half8, bw),
                                                                acc[j & 1], 0, 0, 0);
        }
        const f32x4 dsum = acc[0] + acc[1];
        if (4 * b + g < nchunk) {
            uint32_t scp, mnp;
            q4k_scale_min_pair(hdr.y, hdr.z, hdr.w, g, scp, mnp);
            const float d = doe_half_bits_to_float(hdr.x), dmin = doe_half_bits_to_float(hdr.x >> 16);
            const float qx_lo = (dsum[0] + dsum[1]) * __builtin_amdgcn_ldexpf(1.0f, 24 - sgm[u]);
            const float qx_hi = (dsum[2] + dsum[3]) * __builtin_amdgcn_ldexpf(1.0f, 20 - sgm[u]);
            const float sc_lo = (float)(scp & 0xffu), sc_hi = (float)(scp >> 8);
            const float m_lo = (float)(mnp & 0xffu), m_hi = (float)(mnp >> 8);
            part += d * (sc_lo * qx_lo + sc_hi * qx_hi) - dmin * (m_lo * sxl[u] + m_hi * sxh[u]);
        }
        __builtin_amdgcn_wave_barrier();
    }
    part = sum_rows4(part);  // the row's chunks of this wave's blocks
    if (lane < 16) red[lane * nwaves + wave] = part;
    __syncthreads();

    if (tid < 16) {
        float s = 0.0f;
        for (int j = 0; j < nwaves; ++j) s += red[tid * nwaves + j];
        if (NORM) {
            float tot = 0.0f;
            for (int j = 0; j < nwaves; ++j) tot += ssq[j];
            s *= 1.0f / sqrtf(tot / (float)k + fz.norm_eps);
        }
        const int row = row0 + tid;
        if (fz.gated) {
            const float other = dpp<kDppXor1>(s);  // row ^ 1
            if ((tid & 1) == 0 && row < n) y[row >> 1] = doe_gelu_tanh_clamped(s) * other;
        } else if (ROPE) {
            const float other = dpp<kDppXor1>(s);
            const DoeRopeAhead ra{rope_pos, rope_c, rope_s,
                                  rope_pos >= 0 && rope_pos < fz.max_seq && row < fz.q_rows + fz.kv_rows};
            if ((tid & 1) == 0 && row < n) doe_rope_kv_pair_ahead(rope_kv_of(fz), ra, row, s, other, y);
        } else if (fz.rope_kv) {
            const float other = dpp<kDppXor1>(s);
            if ((tid & 1) == 0 && row < n) rope_kv_pair(fz, row, s, other, y);
        } else if (row < n) {
            const float r = has_res ? s + rpre : s;
            if (fz.y_parts) {
                // the consumer adds the parts; written through (agent scope),
                // so no dirty L2 line is left for the kernel's end to write back
                __hip_atomic_store(fz.y_parts + (size_t)blockIdx.y * n + row, r, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            } else if (gridDim.y > 1) {
                atomicAdd(y + row, s);  // K split: y holds the residual already
            } else {
                y[row] = r;
            }
        }
    }
}

// Streaming form of the matrix-core kernel, for GEMVs of many more 16-row
// groups than CUs: a persistent workgroup of one wave per Q4_K block (nb <=
// 16), or per two blocks (B = 2, nb <= 22: 21-block rows of the 31B-class
// shapes as eleven waves), walks a contiguous range of row groups.  A wave's
// blocks, and so their activation images, are the same in every group: they
// are staged once (the activation parts, if any, added first).  The
// weights go straight from memory into a ring of D LDS slots per wave
// (global_load_lds_dwordx4: lane i's 16 bytes land at slot + 16 i, so granule
// q of a unit -- row q / 9, piece q % 9 -- sits at row * 144 + piece * 16,
// the row layout the MFMA operands are read from, bank-conflict free at that
// stride), so D units per wave stay in flight without holding registers.
// The compiler does not order LDS reads after these loads: each slot is read
// after an explicit vmcnt wait for its three loads (every unit is exactly
// three load instructions, issued unconditionally -- past the range, the last
// group again -- and nothing else reads memory in the walk).  No wave waits
// for another inside the walk: each writes its per-group row partials to
// LDS, and one barrier at the end precedes the cross-wave sums and the
// epilogues.  Measured at 65536 x 2304: 22.8 us against 27.8 for the
// one-shot kernel on the same box, whose workgroups leave their slot empty
// for 1.3-2 us between one workgroup's end and the next one's start.  (One
// ring slot per workgroup, filled with linear 1 KB loads and read after a
// per-group barrier, measured 25.0 us.)
constexpr int kStreamMaxGroups = 16;  // row groups per workgroup (LDS row partials)
constexpr int kStreamMinGroupsPerCu = 8;  // automatic choice: at least 8 row groups per CU
// (two blocks per wave: from 4 -- the one-shot kernel holds one 11-wave
// workgroup per CU there; measured at k 5376: 16384 rows 16.6 against 19.8
// us, 21504 rows 19.4 against 24.3, 43008 rows 31.1 against 45.5)
constexpr int kStreamMinGroupsPerCu2 = 4;
// (the attention-combine prologue over >= 12 blocks per range, or split into
// K ranges: from 2 -- the one-shot form then holds one workgroup per CU
// (78-82 VGPRs); measured at 5376 x 8192, two K ranges, 7 splits: 11.6
// against 16.1 us; four ranges, 6 splits: 9.7 against 12.9)
constexpr int kStreamMinGroupsPerCuAttn = 2;
constexpr int kStreamUnitBytes = 16 * DOE_Q4K_BLOCK_BYTES;  // 16 rows x one block
constexpr int kStreamLdsMax = 160 * 1024;                  // one workgroup per CU
constexpr int kStreamMaxThreads2 = 768;                    // two-block form: at most 12 waves

size_t gemv_stream_lds_bytes(int nwaves, int depth, int bpw = 1) {
    return (size_t)nwaves * bpw * ((size_t)depth * kStreamUnitBytes + kMfmaAImgDwords * 4) +
           (size_t)kStreamMaxGroups * 16 * nwaves * 4 + (size_t)nwaves * 4;
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    // vmcnt N (low 4 bits at [3:0], high 2 at [15:14]), expcnt and lgkmcnt
    // not waited on; the builtin (unlike inline asm) updates the compiler's
    // own count, and the empty asm keeps LDS reads from moving above it
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | (((N >> 4) & 3) << 14));
    __asm__ volatile("" ::: "memory");
}

// (two blocks per wave: at most 11 waves -- the LDS holds no more -- so
// three waves per SIMD and up to 168 VGPRs)
template <int PRO, int XV, int D, int B = 1>
__global__ __launch_bounds__(B == 2 ? kStreamMaxThreads2 : 1024) void q4k_gemv_stream_kernel(
    const uint8_t *__restrict__ w, const float *x, float *__restrict__ y, int n, int k, int nb, int ngroups, int nbs,
    GemvFusion fz) {
    constexpr bool NORM = PRO == 1, ATTN = PRO == 2;
    static_assert(!ATTN || B == 1, "the attention-combine prologue: one block per wave");
    // K range blockIdx.y: blocks [kb0, kb1) (the whole row when not split);
    // a split GEMV writes each range's row sums to its output part
    const int kb0 = (int)blockIdx.y * nbs, kb1 = min(nb, kb0 + nbs);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    // per wave: D ring slots of B units ([16 rows][144] each), then B images
    uint8_t *ring = lds + (size_t)wave * D * B * kStreamUnitBytes;
    uint32_t *aimg = reinterpret_cast<uint32_t *>(lds + (size_t)nwaves * D * B * kStreamUnitBytes +
                                                  (size_t)wave * B * kMfmaAImgDwords * 4);
    float *rpart = reinterpret_cast<float *>(lds + (size_t)nwaves * B * (D * kStreamUnitBytes + kMfmaAImgDwords * 4));
    float *ssq = rpart + kStreamMaxGroups * 16 * nwaves;  // [nwaves]
    // this workgroup's groups [g0, g1): a balanced contiguous split (the host
    // keeps g1 - g0 <= kStreamMaxGroups)
    const int g0 = (int)(((int64_t)blockIdx.x * ngroups) / gridDim.x);
    const int g1 = (int)(((int64_t)blockIdx.x + 1) * ngroups / gridDim.x);
    const int my = g1 - g0;
    const int glast = min(max(g1 - 1, g0), ngroups - 1);

    // Activation (norm weight, activation parts) loads first, then the ring's
    // first loads; the image is built once the activation loads have
    // returned, with the ring's loads still in flight.  Wave w owns
    // blocks B w .. B w + B - 1 (a block past nb reads as zero activations and
    // a clamped copy of the last block's weights).
    float v[B][4], nwv[B][4];
    float4 xp[B][kMaxXParts];
    // the attention prologue's split partials of this lane's four elements
    // (a quad never straddles heads: head_dim % 4 == 0)
    float4 ao[ATTN ? kAttnMaxSplits : 1];
    float2 aml[ATTN ? kAttnMaxSplits : 1];
#pragma unroll
    for (int u = 0; u < B; ++u) {
        const int e = (kb0 + wave * B + u) * 256 + lane * 4;
        if (ATTN) {
            const int S = fz.attn_splits, hd = fz.attn_head_dim;
            const int ec = min(e, k - 4), h = ec / hd, dd = ec - h * hd;
#pragma unroll
            for (int sp = 0; sp < kAttnMaxSplits; ++sp) {
                if (sp < S) {
                    ao[sp] = *reinterpret_cast<const float4 *>(fz.attn_o + ((size_t)h * S + sp) * hd + dd);
                    aml[sp] = *reinterpret_cast<const float2 *>(fz.attn_ml + ((size_t)h * S + sp) * 2);
                }
            }
        } else if (XV) {
            const float4 f = *reinterpret_cast<const float4 *>(x + min(e, k - 4));  // masked below
            v[u][0] = f.x; v[u][1] = f.y; v[u][2] = f.z; v[u][3] = f.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[u][j] = x[min(e + j, k - 1)];
        }
#pragma unroll
        for (int sp = 0; sp < kMaxXParts; ++sp) {
            if (sp < fz.x_nparts) {
                const float *pp = fz.x_parts + (size_t)sp * k;
                if (XV) {
                    xp[u][sp] = *reinterpret_cast<const float4 *>(pp + min(e, k - 4));
                } else {
                    xp[u][sp] = make_float4(pp[min(e, k - 1)], pp[min(e + 1, k - 1)], pp[min(e + 2, k - 1)],
                                            pp[min(e + 3, k - 1)]);
                }
            }
        }
        if (NORM && XV) {
            const float4 f = *reinterpret_cast<const float4 *>(fz.norm_w + min(e, k - 4));
            nwv[u][0] = f.x; nwv[u][1] = f.y; nwv[u][2] = f.z; nwv[u][3] = f.w;
        } else if (NORM) {
#pragma unroll
            for (int j = 0; j < 4; ++j) nwv[u][j] = fz.norm_w[min(e + j, k - 1)];
        }
    }
    const size_t rowbytes = (size_t)nb * DOE_Q4K_BLOCK_BYTES;
    // group gi (clamped to the range), the wave's B blocks, into ring slot d:
    // three load instructions per block (lanes 0..63, 64..127 and 128..143
    // of the 144 granules)
    auto load_unit = [&](int gi, int d) __attribute__((always_inline)) {
        gi = min(gi, glast);
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int bu = min(kb0 + wave * B + u, kb1 - 1);
            uint8_t *slot = ring + (size_t)(d * B + u) * kStreamUnitBytes;
#pragma unroll
            for (int s = 0; s < 3; ++s) {
                const int q = min(lane + 64 * s, 143);
                const int r = min(gi * 16 + q / 9, n - 1);
                const uint8_t *src = w + (size_t)r * rowbytes + (size_t)bu * DOE_Q4K_BLOCK_BYTES + (q % 9) * 16;
                if (s < 2 || lane < 16)
                    __builtin_amdgcn_global_load_lds((const void *)src,
                                                     (__attribute__((address_space(3))) void *)(slot + s * 1024), 16,
                                                     0, 0);
            }
        }
    };
#pragma unroll
    for (int d = 0; d < D; ++d) load_unit(g0 + d, d);
    wait_vmcnt<3 * B * D>();  // the activation loads (older than the ring's) have returned
    if (ATTN) {
        // sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), M = max_s m_s (as the
        // one-shot kernel's prologue)
        const int S = fz.attn_splits;
        float M = -INFINITY;
#pragma unroll
        for (int sp = 0; sp < kAttnMaxSplits; ++sp)
            if (sp < S) M = fmaxf(M, aml[sp].x);
        float L = 0.0f, O0 = 0.0f, O1 = 0.0f, O2 = 0.0f, O3 = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int sp = 0; sp < kAttnMaxSplits; ++sp) {
                if (sp < S) {
                    const float f = exp2f(aml[sp].x - M);
                    L = fmaf(aml[sp].y, f, L);
                    O0 = fmaf(ao[sp].x, f, O0);
                    O1 = fmaf(ao[sp].y, f, O1);
                    O2 = fmaf(ao[sp].z, f, O2);
                    O3 = fmaf(ao[sp].w, f, O3);
                }
            }
        }
        const float rl = L > 0.0f ? 1.0f / L : 0.0f;
        v[0][0] = O0 * rl; v[0][1] = O1 * rl; v[0][2] = O2 * rl; v[0][3] = O3 * rl;
    }

    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < B; ++u) {
        const int e = (kb0 + wave * B + u) * 256 + lane * 4;
        const int e_end = min(k, kb1 * 256);  // past the range: zero (a block of the next range)
#pragma unroll
        for (int sp = 0; sp < kMaxXParts; ++sp) {
            if (sp < fz.x_nparts) {  // x + part 0 + part 1 + ..., in that order
                v[u][0] += xp[u][sp].x; v[u][1] += xp[u][sp].y; v[u][2] += xp[u][sp].z; v[u][3] += xp[u][sp].w;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (e + j >= e_end) v[u][j] = 0.0f;
            if (NORM) {
                ss = fmaf(v[u][j], v[u][j], ss);
                v[u][j] *= fz.norm_offset ? 1.0f + nwv[u][j] : nwv[u][j];
            }
        }
    }
    if (NORM) {
        ss = sum_rows4(sum16(ss));
        if (lane == 0) ssq[wave] = ss;
    }
    // Each block's activation image, staged once (as the one-shot kernel's
    // stage(): lane 16 g + i holds chunk g, quad i).
    const int g = lane >> 4, i16 = lane & 15, m = lane & 15;
    const int nchunk = (k + 63) >> 6;
    float sxl[B], sxh[B], lo_scale[B], hi_scale[B];
    u32x4 areg[B][8];  // the blocks' A operands: the same in every group
#pragma unroll
    for (int u = 0; u < B; ++u) {
        uint32_t *img = aimg + u * kMfmaAImgDwords;
        const float ssum = sum8((v[u][0] + v[u][1]) + (v[u][2] + v[u][3]));
        const float sother = dpp<kDppMirror>(ssum);
        sxl[u] = i16 < 8 ? ssum : sother;
        sxh[u] = i16 < 8 ? sother : ssum;
        float amax = fmaxf(fmaxf(fabsf(v[u][0]), fabsf(v[u][1])), fmaxf(fabsf(v[u][2]), fabsf(v[u][3])));
        amax = fmaxf(amax, dpp<kDppXor1>(amax));
        amax = fmaxf(amax, dpp<kDppXor2>(amax));
        amax = fmaxf(amax, dpp<kDppHalfMirror>(amax));
        amax = fmaxf(amax, dpp<kDppMirror>(amax));
        int sgm = 0;
        if (amax > 0.0f && amax <= 3.0e38f) {
            sgm = 14 - __builtin_amdgcn_frexp_expf(amax);
            sgm = sgm < -100 ? -100 : (sgm > 100 ? 100 : sgm);
        }
        const float xs = __builtin_amdgcn_ldexpf(1.0f, sgm);
        _Float16 hi[4], lo[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float t = v[u][j] * xs;
            hi[j] = (_Float16)t;
            lo[j] = (_Float16)(t - (float)hi[j]);
        }
        const int s = i16 >> 3, jj = i16 & 7;
        const uint32_t h0 = pack_half2(hi[0], hi[2]), h1 = pack_half2(hi[1], hi[3]);
        const uint32_t l0 = pack_half2(lo[0], lo[2]), l1 = pack_half2(lo[1], lo[3]);
        uint32_t *dst = img + jj * kMfmaAStep + g * 16 + s * 4;
        *reinterpret_cast<u32x4 *>(dst) = s ? u32x4{0, 0, h0, h1} : u32x4{h0, h1, 0, 0};
        *reinterpret_cast<u32x4 *>(dst + 8) = s ? u32x4{0, 0, l0, l1} : u32x4{l0, l1, 0, 0};
        if (lane < 8) *reinterpret_cast<u32x4 *>(img + lane * kMfmaAStep + 64) = u32x4{0, 0, 0, 0};
        lo_scale[u] = __builtin_amdgcn_ldexpf(1.0f, 24 - sgm);
        hi_scale[u] = __builtin_amdgcn_ldexpf(1.0f, 20 - sgm);
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int u = 0; u < B; ++u) {
        const int c = 4 * (kb0 + wave * B + u) + g;
        const bool act = (m >> 2) == g && c < nchunk;
        const int abase = act ? g * 16 + (m & 1) * 8 + ((m >> 1) & 1) * 4 : 64;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
            areg[u][jj] = *reinterpret_cast<const u32x4 *>(aimg + u * kMfmaAImgDwords + jj * kMfmaAStep + abase);
    }

    for (int j0 = 0; j0 < my; j0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int j = j0 + d;
            // slot d's 3 B loads are the oldest of the 3 B D in flight
            wait_vmcnt<3 * B * (D - 1)>();
            // The slot's bytes go to registers; the slot is refilled with unit
            // j + D once those reads have returned (before the next unit's
            // bytes may land in it).  Two blocks per wave refill before the
            // arithmetic, so the loads fly during it (31B-class decode +0.3 to
            // +0.8 %, three A/B pairs); one block per wave after it (refilling first
            // measured no faster at 65536 x 2304 and costs 7 VGPRs).
            constexpr bool EARLY = B == 2;
            u32x4 hdr[B], qa[B], qb[B];
            auto read_slot = [&]() __attribute__((always_inline)) {
#pragma unroll
                for (int u = 0; u < B; ++u) {
                    const uint8_t *rp = ring + (size_t)(d * B + u) * kStreamUnitBytes +
                                        i16 * DOE_Q4K_BLOCK_BYTES;  // lane (g, row i16)
                    hdr[u] = *reinterpret_cast<const u32x4 *>(rp);
                    qa[u] = *reinterpret_cast<const u32x4 *>(rp + 16 + 32 * g);
                    qb[u] = *reinterpret_cast<const u32x4 *>(rp + 32 + 32 * g);
                }
            };
            if constexpr (EARLY) {
                if (j < my) read_slot();  // wave-uniform
                __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                load_unit(g0 + j + D, d);
            }
            if (j < my) {  // wave-uniform; LDS and arithmetic only
                if constexpr (!EARLY) read_slot();
                float part = 0.0f;
#pragma unroll
                for (int u = 0; u < B; ++u) {
                    f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        const uint32_t dw = jj < 4 ? qa[u][jj] : qb[u][jj - 4], ew = dw >> 8;
                        const u32x4 bw = {dw & 0x000f000fu, ew & 0x000f000fu, dw & 0x00f000f0u, ew & 0x00f000f0u};
                        acc[jj & 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(half8, areg[u][jj]), __builtin_bit_cast(half8, bw), acc[jj & 1], 0, 0,
                            0);
                    }
                    const f32x4 dsum = acc[0] + acc[1];
                    if (kb0 + wave * B + u < kb1 && 4 * (kb0 + wave * B + u) + g < nchunk) {
                        uint32_t scp, mnp;
                        q4k_scale_min_pair(hdr[u].y, hdr[u].z, hdr[u].w, g, scp, mnp);
                        const float d_ = doe_half_bits_to_float(hdr[u].x);
                        const float dmin = doe_half_bits_to_float(hdr[u].x >> 16);
                        const float qx_lo = (dsum[0] + dsum[1]) * lo_scale[u];
                        const float qx_hi = (dsum[2] + dsum[3]) * hi_scale[u];
                        const float sc_lo = (float)(scp & 0xffu), sc_hi = (float)(scp >> 8);
                        const float m_lo = (float)(mnp & 0xffu), m_hi = (float)(mnp >> 8);
                        part += d_ * (sc_lo * qx_lo + sc_hi * qx_hi) - dmin * (m_lo * sxl[u] + m_hi * sxh[u]);
                    }
                }
                part = sum_rows4(part);
                if (lane < 16) rpart[(j * 16 + lane) * nwaves + wave] = part;
            }
            if constexpr (!EARLY) {
                __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                load_unit(g0 + j + D, d);
            }
        }
    }
    wait_vmcnt<0>();  // the dropped loads past the range land before the LDS is released
    __syncthreads();
    float inv = 1.0f;
    if (NORM) {
        float tot = 0.0f;
        for (int ww = 0; ww < nwaves; ++ww) tot += ssq[ww];
        inv = 1.0f / sqrtf(tot / (float)k + fz.norm_eps);
    }
    auto row_sum = [&](int t) __attribute__((always_inline)) {
        float sm = 0.0f;
        for (int ww = 0; ww < nwaves; ++ww) sm += rpart[t * nwaves + ww];
        return NORM ? sm * inv : sm;
    };
    for (int t = tid; t < my * 16; t += blockDim.x) {
        const int r16 = t & 15;
        const int row = (g0 + (t >> 4)) * 16 + r16;
        if (fz.gated) {
            if ((r16 & 1) == 0 && row < n) y[row >> 1] = doe_gelu_tanh_clamped(row_sum(t)) * row_sum(t + 1);
        } else if (fz.rope_kv) {
            if ((r16 & 1) == 0 && row < n) rope_kv_pair(fz, row, row_sum(t), row_sum(t + 1), y);
        } else if (row < n) {
            const float sv = row_sum(t);
            // the residual (and its parts, added in order) with range 0
            float r = sv;
            if (fz.residual && blockIdx.y == 0) {
                float rs = fz.residual[row];
                for (int sp = 0; sp < fz.res_nparts; ++sp) rs += fz.res_parts[(size_t)sp * n + row];
                r = sv + rs;
            }
            if (fz.y_parts)  // written through (agent scope), as the one-shot kernel's parts
                __hip_atomic_store(fz.y_parts + (size_t)blockIdx.y * n + row, r, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            else
                y[row] = r;
        }
    }
}

// Tunable launch-shape overrides (0 = automatic), set via doe_tune_set.
int g_tune_rowslots = 0;
int g_tune_rows = 0;
int g_tune_kernel = 0;  // 0 automatic, 1 dot-product kernel, 2 matrix-core kernel
int g_tune_ksplit = 0;  // 0 automatic, 1 never split K over workgroups, 2-4: at least that many output parts
int g_tune_forms = 0;   // bits: 1 the q/k/v epilogue without its fetched-ahead rotation,
                        // 2 the attention-prologue o_proj in its fewest K ranges
int g_tune_bpw = 0;     // 0 automatic, else at least this many blocks per wave (<= 4)
int g_tune_stream = 0;  // 0 automatic, -1 never stream, g > 0: stream g row groups per workgroup
int g_tune_stream_depth = 0;  // 0 automatic, else 2, 4 or 6 units in flight per wave (if the LDS allows)

// Launch shape for the GEMV: rowslots * nchunk threads (rounded up to whole
// waves) and R rows per thread.  The automatic choice spreads the rows over
// the CUs in whole workgroups: rows_wg ~ rows per CU / workgroups per CU.
struct GemvShape {
    int rowslots, rows_per_thread, threads;
    size_t lds;
};

size_t gemv_lds_bytes(int nchunk, int rows_wg) {
    return (size_t)nchunk * kLdsChunkDwords * 4 * 2 + (size_t)2 * nchunk * 4 + (size_t)nchunk * 4 +
           (size_t)rows_wg * nchunk * 4 + 16 * 4;
}

GemvShape gemv_shape(int64_t n, int nchunk, int num_cus) {
    // Measured on MI355X (graph replays over 64 rotating weight copies): one
    // row per thread and all of a CU's rows in one workgroup while that stays
    // near 10 waves, otherwise two workgroups per CU (capped at 1024 threads);
    // long rows (k >= 6144) take two rows per thread to amortise the
    // activation staging.  Sweeps at k = 2304 (n = 4096, 9216, 18432), k = 2048
    // and k = 9216 put this rule within 6% of the best shape.
    GemvShape s;
    int max_slots = 1024 / nchunk;
    if (max_slots < 1) max_slots = 1;
    int r = nchunk >= 96 ? 2 : 1;
    if (g_tune_rows == 1 || g_tune_rows == 2 || g_tune_rows == 4) r = g_tune_rows;
    int slots;
    if (g_tune_rowslots > 0) {
        slots = g_tune_rowslots;
    } else {
        const int64_t rows_per_cu = (n + num_cus - 1) / num_cus;
        int64_t want = (rows_per_cu + r - 1) / r;
        if (want * nchunk > 640 && nchunk < 96 && want > 4) want = (want + 1) / 2;
        slots = (int)(want < 4 ? 4 : want);
    }
    if (slots > max_slots) slots = max_slots;
    if (slots < 1) slots = 1;
    s.rowslots = slots;
    s.rows_per_thread = r;
    s.threads = ((slots * nchunk + 63) / 64) * 64;
    s.lds = gemv_lds_bytes(nchunk, slots * r);
    return s;
}

int g_num_cus = 0;

}  // namespace

extern "C" {

int doe_q4k_dequant(const void *weight_q4k, float *out, int64_t n, int64_t k,
                    doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(n >= 0 && k >= 0, DOE_E_INVALID, "negative shape n=%lld k=%lld", (long long)n,
                (long long)k);
    if (n == 0 || k == 0) return DOE_OK;
    DOE_REQUIRE(weight_q4k && out, DOE_E_INVALID, "null pointer");
    DOE_REQUIRE(((uintptr_t)weight_q4k & 15) == 0, DOE_E_INVALID, "weight must be 16-byte aligned");
    const int64_t nb = (k + 255) / 256;
    const int64_t total = n * nb * 128;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(q4k_dequant_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, (const uint8_t *)weight_q4k, out, n, k, nb);
    DOE_LAUNCH_CHECK("q4k_dequant_kernel");
    return DOE_OK;
}

}  // extern "C"

namespace {

// max_y_parts / y_nparts: with fz.y_parts, the most K ranges the caller's
// parts buffer holds and where the number used is returned.
int gemv_launch(const void *weight_q4k, const float *activation, float *output, int64_t n,
                int64_t k, const GemvFusion &fz, hipStream_t st, int max_y_parts = 0,
                int32_t *y_nparts = nullptr) {
    int rc = doe::require_init();
    if (rc) return rc;
    const bool xparts = fz.x_nparts > 0;
    DOE_REQUIRE(fz.x_nparts >= 0 && fz.x_nparts <= kMaxXParts && (!xparts || fz.x_parts), DOE_E_INVALID,
                "activation parts: 0..%d with a parts pointer (got %d)", kMaxXParts, fz.x_nparts);
    DOE_REQUIRE(!xparts || !fz.attn_o, DOE_E_UNSUPPORTED, "activation parts exclude the attention prologue");
    DOE_REQUIRE(!fz.y_parts || (!fz.gated && !fz.rope_kv && !fz.norm_w && y_nparts && max_y_parts >= 1),
                DOE_E_UNSUPPORTED, "output parts: plain, residual or attention-prologue GEMVs, a count pointer "
                                   "and room for at least one part");
    DOE_REQUIRE(n >= 0 && k >= 0, DOE_E_INVALID, "negative shape n=%lld k=%lld", (long long)n,
                (long long)k);
    DOE_REQUIRE(!fz.gated || (n % 2) == 0, DOE_E_INVALID, "gated GEMV needs an even row count");
    DOE_REQUIRE(!(fz.gated && fz.rope_kv) && !(fz.rope_kv && fz.residual), DOE_E_UNSUPPORTED,
                "rope/kv epilogue excludes gated and residual");
    DOE_REQUIRE(!(fz.gated && fz.residual), DOE_E_UNSUPPORTED, "gated and residual are exclusive");
    DOE_REQUIRE(fz.res_nparts >= 0 && fz.res_nparts <= kMaxXParts &&
                    (fz.res_nparts == 0 || (fz.res_parts && fz.residual)),
                DOE_E_INVALID, "residual parts: 0..%d with a residual and a parts pointer (got %d)", kMaxXParts,
                fz.res_nparts);
    DOE_REQUIRE(fz.res_nparts == 0 || (fz.residual != output && !fz.norm_w), DOE_E_UNSUPPORTED,
                "residual parts need an output apart from the residual and no RMSNorm prologue");
    if (n == 0) return DOE_OK;
    DOE_REQUIRE(output, DOE_E_INVALID, "null output");
    if (k == 0) {
        // Empty reduction: the sum identity (reference_interpreter.zig:323-327).
        DOE_REQUIRE(!fz.residual && !fz.gated, DOE_E_UNSUPPORTED, "fused epilogues need k > 0");
        if (fz.y_parts) {
            *y_nparts = 1;
            return doe::fill_bytes_async(fz.y_parts, 0, (size_t)n * sizeof(float), st);
        }
        return doe::fill_bytes_async(output, 0, (size_t)n * sizeof(float), st);
    }
    DOE_REQUIRE(weight_q4k && (activation || fz.attn_o), DOE_E_INVALID, "null pointer");
    DOE_REQUIRE(((uintptr_t)weight_q4k & 15) == 0, DOE_E_INVALID, "weight must be 16-byte aligned");
    DOE_REQUIRE(n <= 0x7fffffff && k <= 65536, DOE_E_UNSUPPORTED,
                "q4k_gemv supports n < 2^31 and k <= 65536 (got n=%lld k=%lld)", (long long)n,
                (long long)k);
    const int nb = (int)((k + 255) / 256);
    const int nchunk = (int)((k + 63) / 64);
    const uint8_t *wp = (const uint8_t *)weight_q4k;
    // Matrix-core kernel, up to 64 blocks per workgroup (up to four per wave;
    // the attention-combine prologue is single-block) and K split beyond;
    // measured faster than the dot-product kernel on every decode shape.
    // `q4k_gemv.kernel` = 1 forces the dot-product kernel where its LDS holds
    // the activation (k <~ 12K).
    if (g_num_cus == 0) {
        int dev = 0, cus = 0;
        DOE_HIP_CHECK(hipGetDevice(&dev));
        DOE_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        g_num_cus = cus > 0 ? cus : 256;
    }
    // K split over workgroups (at most 16 blocks, one per wave, each), the
    // partial row sums added atomically into y: only for an in-place residual
    // (y already holds it) and an element-wise activation prologue (not the
    // RMSNorm, whose scale needs the whole row), when the rows alone give
    // fewer workgroups than CUs.
    const int64_t row_groups = (n + 15) / 16;
    int ksplit = 1;
    if (nb > kMfmaMaxBlocks) {
        // Past 64 blocks a row no longer fits one workgroup: K ranges of at
        // most 16 blocks (one per wave) add their row sums atomically into y,
        // which starts at the residual (or zero).  The fused prologues and
        // epilogues need whole rows.
        DOE_REQUIRE(!fz.norm_w && !fz.gated && !fz.rope_kv && !fz.attn_o, DOE_E_UNSUPPORTED,
                    "k=%lld (%d Q4_K blocks > %d): only the plain and residual forms", (long long)k, nb,
                    kMfmaMaxBlocks);
        if (fz.y_parts) {
            // K ranges of at most 64 blocks, each written to its own part
            ksplit = (nb + kMfmaMaxBlocks - 1) / kMfmaMaxBlocks;
            DOE_REQUIRE(ksplit <= max_y_parts && ksplit <= kMaxXParts, DOE_E_UNSUPPORTED,
                        "k=%lld needs %d output parts (room for %d, at most %d)", (long long)k, ksplit,
                        max_y_parts, kMaxXParts);
            const int64_t fill = (g_num_cus + row_groups - 1) / row_groups;  // more ranges while CUs idle
            int want = (int)(fill < nb ? fill : nb);
            if (want < (nb + 15) / 16) want = (nb + 15) / 16;
            if (want > max_y_parts) want = max_y_parts;
            if (want > kMaxXParts) want = kMaxXParts;
            if (want > ksplit && g_tune_ksplit != 1) ksplit = want;
        } else if (fz.residual && fz.residual != output) {
            DOE_HIP_CHECK(hipMemcpyAsync(output, fz.residual, (size_t)n * sizeof(float), hipMemcpyDeviceToDevice, st));
        } else if (!fz.residual) {
            rc = doe::fill_bytes_async(output, 0, (size_t)n * sizeof(float), st);
            if (rc) return rc;
        }
        if (!fz.y_parts) ksplit = (nb + 15) / 16;
    } else if (fz.y_parts) {
        // K ranges while the rows alone leave CUs idle, one block per wave
        // where the parts allow; each range writes its own part.  The
        // attention prologue is single-block: at least one range per 16 blocks.
        const int cap = max_y_parts < kMaxXParts ? max_y_parts : kMaxXParts;
        const int need = fz.attn_o ? (nb + 15) / 16 : 1;
        ksplit = need;
        // past 16 blocks the attention prologue takes as many K ranges as the
        // parts allow: fewer blocks per range, each wave walking more row
        // groups (5376 x 8192, six splits of 32 heads: four ranges of 8
        // blocks 9.7 us against 10.7 for two of 16, same buffers)
        if (need > 1 && !(g_tune_forms & 2)) ksplit = cap < nb ? cap : nb;
        if (row_groups < g_num_cus && g_tune_ksplit != 1 && nb > 1) {
            const int64_t fill = (g_num_cus + row_groups - 1) / row_groups;
            int want = (int)(fill < nb ? fill : nb);
            if (want < (nb + 15) / 16) want = (nb + 15) / 16;
            if (want > cap) want = cap;
            if (want > ksplit) ksplit = want;
        }
        if (g_tune_ksplit > ksplit) ksplit = (int)(g_tune_ksplit < cap ? (g_tune_ksplit < nb ? g_tune_ksplit : nb) : cap);
        DOE_REQUIRE(ksplit <= cap, DOE_E_UNSUPPORTED, "k=%lld needs %d output parts (room for %d, at most %d)",
                    (long long)k, ksplit, max_y_parts, kMaxXParts);
    } else if (nb > 1 && fz.residual == output && !fz.norm_w && !fz.gated && !fz.rope_kv &&
               row_groups < g_num_cus && g_tune_ksplit != 1) {
        const int64_t fill = (g_num_cus + row_groups - 1) / row_groups;
        ksplit = (int)(fill < nb ? fill : nb);
        if (ksplit < (nb + 15) / 16) ksplit = (nb + 15) / 16;
    }
    if (fz.y_parts) *y_nparts = ksplit;
    const int nbs = (nb + ksplit - 1) / ksplit;  // blocks per split
    int bpw = nbs <= 16 ? 1 : (nbs <= 32 ? 2 : (nbs <= 48 ? 3 : 4));
    if (g_tune_bpw > bpw && g_tune_bpw <= 4 && !fz.attn_o) bpw = g_tune_bpw;
    const bool mfma_ok = nbs <= kMfmaMaxBlocks && (bpw == 1 || !fz.attn_o);
    const bool dot_ok = gemv_lds_bytes(nchunk, 8) <= 64 * 1024;
    const bool use_mfma = g_tune_kernel == 1 ? !dot_ok && mfma_ok : mfma_ok;
    // Streaming kernel: one wave per block, whole rows, no attention
    // prologue; automatic from kStreamMinGroupsPerCu row groups per CU
    // (q4k_gemv.stream: -1 never, g > 0 forces g row groups per workgroup).
    DOE_REQUIRE(!(xparts || fz.y_parts || fz.res_nparts) || use_mfma, DOE_E_UNSUPPORTED,
                "activation / output / residual parts need the matrix-core kernel");
    DOE_REQUIRE(!fz.res_nparts || ksplit == 1 || fz.y_parts, DOE_E_UNSUPPORTED,
                "residual parts need whole rows or output parts");
    DOE_REQUIRE(!xparts || bpw <= 2, DOE_E_UNSUPPORTED,
                "activation parts need k <= 8192 (two Q4_K blocks per wave; got k=%lld)", (long long)k);
    DOE_REQUIRE(!fz.x_sum || ksplit == 1, DOE_E_UNSUPPORTED, "the activation sum needs whole rows");
    // (two blocks per wave while the ring and images fit the LDS: k <= 22
    // blocks; activation parts summed in its prologue, the sum not kept)
    // (two blocks per wave while the ring and images fit the LDS: up to 22
    // blocks per row or K range; activation parts summed in its prologue,
    // the sum not kept; K ranges only as output parts)
    const bool stream_ok = use_mfma && (bpw == 1 || (bpw == 2 && gemv_stream_lds_bytes((nbs + 1) / 2, 2, 2) <=
                                                                      (size_t)kStreamLdsMax)) &&
                           (ksplit == 1 || fz.y_parts) && (!fz.attn_o || bpw == 1) && !fz.x_sum;
    const int stream_min = bpw == 2                       ? kStreamMinGroupsPerCu2
                           : (fz.attn_o && (nbs >= 12 || ksplit > 1)) ? kStreamMinGroupsPerCuAttn
                                                      : kStreamMinGroupsPerCu;
    if (stream_ok &&
        (g_tune_stream > 0 || (g_tune_stream == 0 && row_groups * ksplit >= (int64_t)stream_min * g_num_cus))) {
        const int sb = bpw;  // blocks per wave
        const int nwaves = (nbs + sb - 1) / sb;
        DOE_REQUIRE(sb == 1 || 64 * nwaves <= kStreamMaxThreads2, DOE_E_UNSUPPORTED,
                    "two-block streaming GEMV: %d waves (at most %d)", nwaves, kStreamMaxThreads2 / 64);
        // ring depth 2: deeper rings measured slower (65536 x 2304: 21.4 us
        // at 2, 23.0 at 3, 23.4 at 4, 25.8 at 6) -- the more units each wave
        // has in flight, the further a workgroup's waves drift apart over
        // the groups and the less DRAM row locality their reads keep
        int depth = 2;
        if (sb == 1 && g_tune_stream_depth > 0 && gemv_stream_lds_bytes(nwaves, g_tune_stream_depth) <= kStreamLdsMax)
            depth = g_tune_stream_depth;
        const size_t lds = gemv_stream_lds_bytes(nwaves, depth, sb);
        const bool xv = ((uintptr_t)activation & 15) == 0 && (k & 3) == 0 && ((uintptr_t)fz.norm_w & 15) == 0 &&
                        ((uintptr_t)fz.x_parts & 15) == 0;
        static const hipError_t attr_all = [] {
            hipError_t e = hipSuccess;
            for (const void *f : {(const void *)q4k_gemv_stream_kernel<0, 0, 2>, (const void *)q4k_gemv_stream_kernel<0, 1, 2>,
                                  (const void *)q4k_gemv_stream_kernel<1, 0, 2>, (const void *)q4k_gemv_stream_kernel<1, 1, 2>,
                                  (const void *)q4k_gemv_stream_kernel<0, 0, 4>, (const void *)q4k_gemv_stream_kernel<0, 1, 4>,
                                  (const void *)q4k_gemv_stream_kernel<1, 0, 4>, (const void *)q4k_gemv_stream_kernel<1, 1, 4>,
                                  (const void *)q4k_gemv_stream_kernel<0, 0, 6>, (const void *)q4k_gemv_stream_kernel<0, 1, 6>,
                                  (const void *)q4k_gemv_stream_kernel<1, 0, 6>, (const void *)q4k_gemv_stream_kernel<1, 1, 6>,
                                  (const void *)q4k_gemv_stream_kernel<0, 0, 3>, (const void *)q4k_gemv_stream_kernel<0, 1, 3>,
                                  (const void *)q4k_gemv_stream_kernel<1, 0, 3>, (const void *)q4k_gemv_stream_kernel<1, 1, 3>,
                                  (const void *)q4k_gemv_stream_kernel<0, 0, 2, 2>, (const void *)q4k_gemv_stream_kernel<0, 1, 2, 2>,
                                  (const void *)q4k_gemv_stream_kernel<1, 0, 2, 2>, (const void *)q4k_gemv_stream_kernel<1, 1, 2, 2>,
                                  (const void *)q4k_gemv_stream_kernel<2, 0, 2, 1>})
                if (e == hipSuccess) e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kStreamLdsMax);
            return e;
        }();
        DOE_HIP_CHECK(attr_all);
        // groups per workgroup: forced, or one workgroup per CU (LDS-bound)
        // over the row groups of every K range, at most kStreamMaxGroups each
        // (two workgroups per CU of half the groups measured slower with the
        // same buffers: 65536 x 2304 22.9 against 20.0 us, 32768 x 2304 14.2
        // against 12.3)
        int64_t per_wg = g_tune_stream > 0 ? g_tune_stream : (row_groups * ksplit + g_num_cus - 1) / g_num_cus;
        if (per_wg > kStreamMaxGroups) per_wg = kStreamMaxGroups;
        const int64_t grid = (row_groups + per_wg - 1) / per_wg;
        const dim3 sgrid((unsigned)grid, (unsigned)ksplit);
#define DOE_GEMV_STREAM_LAUNCH(P, X, D)                                                                   \
    hipLaunchKernelGGL((q4k_gemv_stream_kernel<P, X, D>), sgrid, dim3(64 * nwaves), lds, st, wp, activation, output, \
                       (int)n, (int)k, nb, (int)row_groups, nbs, fz)
#define DOE_GEMV_STREAM_DEPTH(P, X)                                                                       \
    do {                                                                                                  \
        if (sb == 2)                                                                                      \
            hipLaunchKernelGGL((q4k_gemv_stream_kernel<P, X, 2, 2>), sgrid, dim3(64 * nwaves), lds, st, wp,      \
                               activation, output, (int)n, (int)k, nb, (int)row_groups, nbs, fz);        \
        else if (depth == 4) DOE_GEMV_STREAM_LAUNCH(P, X, 4);                                            \
        else if (depth == 6) DOE_GEMV_STREAM_LAUNCH(P, X, 6);                                            \
        else if (depth == 3) DOE_GEMV_STREAM_LAUNCH(P, X, 3);                                            \
        else DOE_GEMV_STREAM_LAUNCH(P, X, 2);                                                            \
    } while (0)
        if (fz.attn_o) {
            hipLaunchKernelGGL((q4k_gemv_stream_kernel<2, 0, 2, 1>), sgrid, dim3(64 * nwaves), lds, st, wp, activation,
                               output, (int)n, (int)k, nb, (int)row_groups, nbs, fz);
        } else if (fz.norm_w) {
            if (xv) DOE_GEMV_STREAM_DEPTH(1, 1); else DOE_GEMV_STREAM_DEPTH(1, 0);
        } else {
            if (xv) DOE_GEMV_STREAM_DEPTH(0, 1); else DOE_GEMV_STREAM_DEPTH(0, 0);
        }
#undef DOE_GEMV_STREAM_DEPTH
#undef DOE_GEMV_STREAM_LAUNCH
        DOE_LAUNCH_CHECK("q4k_gemv_stream_kernel");
        return DOE_OK;
    }
    if (use_mfma) {
        const int nwaves = (nbs + bpw - 1) / bpw;
        const size_t lds = gemv_mfma_lds_bytes(nwaves, bpw);
        const dim3 grid((unsigned)row_groups, (unsigned)ksplit);
        const bool xv = activation && ((uintptr_t)activation & 15) == 0 && (k & 3) == 0 &&
                        ((uintptr_t)fz.norm_w & 15) == 0 && ((uintptr_t)fz.x_parts & 15) == 0;
#define DOE_GEMV_MFMA_LAUNCH(P, B, X, R)                                                             \
    do {                                                                                          \
        /* set once per process; a static's initialisation is thread-safe */                    \
        static const hipError_t attr_rc = hipFuncSetAttribute(                                    \
            (const void *)q4k_gemv_mfma_kernel<P, B, X, R>, hipFuncAttributeMaxDynamicSharedMemorySize, \
            (int)gemv_mfma_lds_bytes(16, B));                                                     \
        DOE_HIP_CHECK(attr_rc);                                                                   \
        hipLaunchKernelGGL((q4k_gemv_mfma_kernel<P, B, X, R>), grid, dim3(64 * nwaves), lds, st, wp, \
                           activation, output, (int)n, (int)k, nb, nbs, fz);                      \
    } while (0)
#define DOE_GEMV_MFMA_BPW(P, X, R)                                                                   \
    switch (bpw) {                                                                                \
        case 1: DOE_GEMV_MFMA_LAUNCH(P, 1, X, R); break;                                             \
        case 2: DOE_GEMV_MFMA_LAUNCH(P, 2, X, R); break;                                             \
        case 3: DOE_GEMV_MFMA_LAUNCH(P, 3, X, R); break;                                             \
        default: DOE_GEMV_MFMA_LAUNCH(P, 4, X, R); break;                                            \
    }
        if (fz.attn_o && fz.res_nparts) {
            DOE_GEMV_MFMA_LAUNCH(2, 1, 0, 1);
        } else if (fz.attn_o) {
            DOE_GEMV_MFMA_LAUNCH(2, 1, 0, 0);
        } else if (fz.norm_w && fz.rope_kv && bpw == 1 && xv && !(g_tune_forms & 1)) {
            DOE_GEMV_MFMA_LAUNCH(1, 1, 1, 2);  // the decode step's q/k/v projection
        } else if (fz.norm_w) {
            if (xv) DOE_GEMV_MFMA_BPW(1, 1, 0) else DOE_GEMV_MFMA_BPW(1, 0, 0)
        } else if (fz.res_nparts) {
            if (xv) DOE_GEMV_MFMA_BPW(0, 1, 1) else DOE_GEMV_MFMA_BPW(0, 0, 1)
        } else {
            if (xv) DOE_GEMV_MFMA_BPW(0, 1, 0) else DOE_GEMV_MFMA_BPW(0, 0, 0)
        }
#undef DOE_GEMV_MFMA_BPW
#undef DOE_GEMV_MFMA_LAUNCH
        DOE_LAUNCH_CHECK("q4k_gemv_mfma_kernel");
        return DOE_OK;
    }
    GemvShape s = gemv_shape(n, nchunk, g_num_cus);
    if ((fz.gated || fz.rope_kv) && ((s.rowslots * s.rows_per_thread) & 1)) {
        // a gate/up row pair must not straddle two workgroups
        if (s.rowslots + 1 <= 1024 / nchunk) s.rowslots += 1;
        else if (s.rowslots > 1) s.rowslots -= 1;
        else s.rows_per_thread = 2;
        s.threads = ((s.rowslots * nchunk + 63) / 64) * 64;
        s.lds = gemv_lds_bytes(nchunk, s.rowslots * s.rows_per_thread);
    }
    DOE_REQUIRE(s.lds <= 64 * 1024, DOE_E_UNSUPPORTED, "k=%lld needs %zu bytes of LDS",
                (long long)k, s.lds);
    const int rows_wg = s.rowslots * s.rows_per_thread;
    const unsigned grid = (unsigned)((n + rows_wg - 1) / rows_wg);
    const int nquads = nchunk * 16;
    const int q = (nquads + s.threads - 1) / s.threads;
    DOE_REQUIRE((!fz.norm_w && !fz.attn_o) || q <= 4, DOE_E_UNSUPPORTED,
                "fused RMSNorm / attention combine needs k <= %d here", 4 * s.threads * 4);
    const int qsel = q <= 1 ? 1 : (q <= 2 ? 2 : 4);
#define DOE_GEMV_LAUNCH(RR, QQ)                                                                  \
    if (fz.attn_o)                                                                                \
        hipLaunchKernelGGL((q4k_gemv_kernel<RR, QQ, 2>), dim3(grid), dim3(s.threads), s.lds,     \
                           st, wp, activation, output, (int)n, (int)k, nb, nchunk, s.rowslots, fz); \
    else if (fz.norm_w)                                                                           \
        hipLaunchKernelGGL((q4k_gemv_kernel<RR, QQ, 1>), dim3(grid), dim3(s.threads), s.lds,     \
                           st, wp, activation, output, (int)n, (int)k, nb, nchunk, s.rowslots, fz); \
    else                                                                                          \
        hipLaunchKernelGGL((q4k_gemv_kernel<RR, QQ, 0>), dim3(grid), dim3(s.threads), s.lds,     \
                           st, wp, activation, output, (int)n, (int)k, nb, nchunk, s.rowslots, fz)
    switch (s.rows_per_thread * 8 + qsel) {
        case 1 * 8 + 1: DOE_GEMV_LAUNCH(1, 1); break;
        case 1 * 8 + 2: DOE_GEMV_LAUNCH(1, 2); break;
        case 1 * 8 + 4: DOE_GEMV_LAUNCH(1, 4); break;
        case 2 * 8 + 1: DOE_GEMV_LAUNCH(2, 1); break;
        case 2 * 8 + 2: DOE_GEMV_LAUNCH(2, 2); break;
        case 2 * 8 + 4: DOE_GEMV_LAUNCH(2, 4); break;
        case 4 * 8 + 1: DOE_GEMV_LAUNCH(4, 1); break;
        case 4 * 8 + 2: DOE_GEMV_LAUNCH(4, 2); break;
        default: DOE_GEMV_LAUNCH(4, 4); break;
    }
#undef DOE_GEMV_LAUNCH
    DOE_LAUNCH_CHECK("q4k_gemv_kernel");
    return DOE_OK;
}

}  // namespace

extern "C" {

int doe_q4k_gemv(const void *weight_q4k, const float *activation, float *output, int64_t n,
                 int64_t k, doe_stream_t stream) {
    GemvFusion fz{};
    return gemv_launch(weight_q4k, activation, output, n, k, fz, (hipStream_t)stream);
}

int doe_q4k_gemv_fused(const void *weight_q4k, const float *activation, float *output, int64_t n,
                       int64_t k, const float *norm_weight, float norm_eps, int norm_weight_offset,
                       const float *residual, int gated, doe_stream_t stream) {
    GemvFusion fz{};
    fz.norm_w = norm_weight;
    fz.norm_eps = norm_eps;
    fz.norm_offset = norm_weight_offset;
    fz.residual = residual;
    fz.gated = gated;
    return gemv_launch(weight_q4k, activation, output, n, k, fz, (hipStream_t)stream);
}

int doe_q4k_gemv_qkv_rope_kv(const void *weight_q4k, const float *activation, float *output,
                             int64_t hidden, const float *norm_weight, float norm_eps,
                             int norm_weight_offset, int64_t num_heads, int64_t num_kv_heads,
                             int64_t head_dim, const float *freq_cis, const int32_t *position_dev,
                             uint16_t *key_cache, uint16_t *val_cache, int64_t max_seq_len,
                             doe_stream_t stream) {
    DOE_REQUIRE(num_heads > 0 && num_kv_heads >= 0 && head_dim > 0 && (head_dim % 2) == 0 &&
                    max_seq_len > 0,
                DOE_E_INVALID, "bad qkv shape");
    // num_kv_heads 0: the q rows alone (a layer that reads another layer's
    // KV cache), no cache row is written and the caches may be NULL
    DOE_REQUIRE(freq_cis && position_dev && (num_kv_heads == 0 || (key_cache && val_cache)), DOE_E_INVALID,
                "null pointer");
    GemvFusion fz{};
    fz.norm_w = norm_weight;
    fz.norm_eps = norm_eps;
    fz.norm_offset = norm_weight_offset;
    fz.rope_kv = 1;
    fz.freq_cis = freq_cis;
    fz.pos_dev = position_dev;
    fz.k_cache = (_Float16 *)key_cache;
    fz.v_cache = (_Float16 *)val_cache;
    fz.q_rows = (int)(num_heads * head_dim);
    fz.kv_rows = (int)(num_kv_heads * head_dim);
    fz.head_dim = (int)head_dim;
    fz.max_seq = (int)max_seq_len;
    const int64_t n = (num_heads + 2 * num_kv_heads) * head_dim;
    return gemv_launch(weight_q4k, activation, output, n, hidden, fz, (hipStream_t)stream);
}

int doe_q4k_gemv_attn_out(const void *weight_q4k, const float *attn_partials, int64_t splits,
                          int64_t num_heads, int64_t head_dim, float *output, int64_t n,
                          const float *residual, doe_stream_t stream) {
    DOE_REQUIRE(attn_partials, DOE_E_INVALID, "null partials");
    DOE_REQUIRE(splits >= 1 && splits <= kAttnMaxSplits, DOE_E_UNSUPPORTED,
                "attention combine prologue supports 1..%d splits (got %lld)", kAttnMaxSplits,
                (long long)splits);
    DOE_REQUIRE(num_heads > 0 && head_dim > 0 && head_dim % 4 == 0, DOE_E_INVALID, "bad head shape");
    DOE_REQUIRE(((uintptr_t)attn_partials & 15) == 0, DOE_E_INVALID, "partials must be 16-byte aligned");
    GemvFusion fz{};
    fz.attn_o = attn_partials;
    fz.attn_ml = attn_partials + num_heads * splits * head_dim;
    fz.attn_splits = (int)splits;
    fz.attn_head_dim = (int)head_dim;
    fz.residual = residual;
    return gemv_launch(weight_q4k, nullptr, output, n, num_heads * head_dim, fz, (hipStream_t)stream);
}

int doe_q4k_gemv_ex(const doe_q4k_gemv_args *a, doe_stream_t stream) {
    DOE_REQUIRE(a, DOE_E_INVALID, "null arguments");
    DOE_REQUIRE(a->activation_nparts >= 0 && a->activation_nparts <= kMaxXParts, DOE_E_INVALID,
                "activation_nparts %lld (0..%d)", (long long)a->activation_nparts, kMaxXParts);
    DOE_REQUIRE(!a->activation_sum || a->activation_nparts > 0, DOE_E_INVALID,
                "activation_sum without activation parts");
    DOE_REQUIRE(!a->output_parts || (a->output_nparts && a->max_output_parts >= 1 && a->max_output_parts < 1024),
                DOE_E_INVALID, "output_parts needs output_nparts and 1 <= max_output_parts");
    GemvFusion fz{};
    fz.norm_w = a->norm_weight;
    fz.norm_eps = a->norm_eps;
    fz.norm_offset = a->norm_weight_offset;
    fz.residual = a->residual;
    fz.gated = a->gated;
    fz.res_parts = a->residual_parts;
    fz.res_nparts = (int)a->residual_nparts;
    DOE_REQUIRE(a->residual_nparts >= 0 && a->residual_nparts <= kMaxXParts, DOE_E_INVALID,
                "residual_nparts %lld (0..%d)", (long long)a->residual_nparts, kMaxXParts);
    fz.x_parts = a->activation_parts;
    fz.x_nparts = (int)a->activation_nparts;
    fz.x_sum = a->activation_sum;
    fz.y_parts = a->output_parts;
    int64_t n = a->n, k = a->k;
    if (a->rope_kv) {
        DOE_REQUIRE(a->num_heads > 0 && a->num_kv_heads >= 0 && a->head_dim > 0 && (a->head_dim % 2) == 0 &&
                        a->max_seq_len > 0,
                    DOE_E_INVALID, "bad qkv shape");
        DOE_REQUIRE(a->freq_cis && a->position_dev && (a->num_kv_heads == 0 || (a->key_cache && a->val_cache)),
                    DOE_E_INVALID, "null pointer");
        DOE_REQUIRE(n == (a->num_heads + 2 * a->num_kv_heads) * a->head_dim, DOE_E_INVALID,
                    "n %lld is not (num_heads + 2 num_kv_heads) x head_dim", (long long)n);
        fz.rope_kv = 1;
        fz.freq_cis = a->freq_cis;
        fz.pos_dev = a->position_dev;
        fz.k_cache = (_Float16 *)a->key_cache;
        fz.v_cache = (_Float16 *)a->val_cache;
        fz.q_rows = (int)(a->num_heads * a->head_dim);
        fz.kv_rows = (int)(a->num_kv_heads * a->head_dim);
        fz.head_dim = (int)a->head_dim;
        fz.max_seq = (int)a->max_seq_len;
    }
    if (a->attn_partials) {
        DOE_REQUIRE(a->attn_splits >= 1 && a->attn_splits <= kAttnMaxSplits, DOE_E_UNSUPPORTED,
                    "attention combine prologue supports 1..%d splits (got %lld)", kAttnMaxSplits,
                    (long long)a->attn_splits);
        DOE_REQUIRE(a->attn_num_heads > 0 && a->attn_head_dim > 0 && a->attn_head_dim % 4 == 0, DOE_E_INVALID,
                    "bad head shape");
        DOE_REQUIRE(((uintptr_t)a->attn_partials & 15) == 0, DOE_E_INVALID, "partials must be 16-byte aligned");
        DOE_REQUIRE(!a->activation && k == a->attn_num_heads * a->attn_head_dim, DOE_E_INVALID,
                    "with attn_partials the activation is NULL and k = num_heads x head_dim");
        fz.attn_o = a->attn_partials;
        fz.attn_ml = a->attn_partials + a->attn_num_heads * a->attn_splits * a->attn_head_dim;
        fz.attn_splits = (int)a->attn_splits;
        fz.attn_head_dim = (int)a->attn_head_dim;
    }
    float *out = a->output;
    if (a->output_parts && !out) out = a->output_parts;  // (unused: the parts are the output)
    return gemv_launch(a->weight_q4k, a->activation, out, n, k, fz, (hipStream_t)stream,
                       (int)a->max_output_parts, a->output_nparts);
}

int doe_tune_set(const char *key, int value) {
    DOE_REQUIRE(key, DOE_E_INVALID, "null key");
    if (!strcmp(key, "q4k_gemv.rowslots")) {
        g_tune_rowslots = value;
    } else if (!strcmp(key, "q4k_gemv.rows")) {
        g_tune_rows = value;
    } else if (!strcmp(key, "q4k_gemv.bpw")) {
        DOE_REQUIRE(value >= 0 && value <= 4, DOE_E_INVALID, "q4k_gemv.bpw is 0..4");
        g_tune_bpw = value;
    } else if (!strcmp(key, "q4k_gemv.stream")) {
        DOE_REQUIRE(value >= -1 && value <= kStreamMaxGroups, DOE_E_INVALID, "q4k_gemv.stream is -1..%d",
                    kStreamMaxGroups);
        g_tune_stream = value;
    } else if (!strcmp(key, "q4k_gemv.stream_depth")) {
        DOE_REQUIRE(value == 0 || value == 2 || value == 3 || value == 4 || value == 6, DOE_E_INVALID,
                    "q4k_gemv.stream_depth is 0, 2, 3, 4 or 6");
        g_tune_stream_depth = value;
    } else if (!strcmp(key, "q4k_gemv.ksplit")) {
        DOE_REQUIRE(value >= 0 && value <= kMaxXParts, DOE_E_INVALID, "q4k_gemv.ksplit is 0..%d", kMaxXParts);
        g_tune_ksplit = value;
    } else if (!strcmp(key, "q4k_gemv.forms")) {
        DOE_REQUIRE(value >= 0 && value <= 3, DOE_E_INVALID, "q4k_gemv.forms is 0..3");
        g_tune_forms = value;
    } else if (!strcmp(key, "q4k_gemv.kernel")) {
        DOE_REQUIRE(value >= 0 && value <= 2, DOE_E_INVALID, "q4k_gemv.kernel is 0, 1 or 2");
        g_tune_kernel = value;
    } else if (!strcmp(key, "q8_0_gemv.rows") || !strcmp(key, "q8_0_gemv.depth")) {
        return doe::q8_0_set_tune(key, value);
    } else if (!strcmp(key, "int4_gemv.kernel")) {
        return doe::int4_set_kernel(value);
    } else if (!strcmp(key, "int4_gemv.depth")) {
        return doe::int4_set_depth(value);
    } else if (!strcmp(key, "int4_gemv.xcd")) {
        return doe::int4_set_xcd(value);
    } else if (!strcmp(key, "attn_mq.splits")) {
        return doe::mq_set_splits(value);
    } else if (!strcmp(key, "attn_decode.splits")) {
        return doe::attn_set_splits(value);
    } else if (!strcmp(key, "attn_decode.waves")) {
        return doe::attn_set_waves(value);
    } else if (!strcmp(key, "attn_decode.combine")) {
        return doe::attn_set_combine(value);
    } else if (!strcmp(key, "quant_gemm.f16_operands")) {
        return doe::gemm_set_f16_operands(value);
    } else {
        return doe::set_error(DOE_E_INVALID, "unknown tuning key '%s'", key);
    }
    return DOE_OK;
}

}  // extern "C"
