// q8_0_gemv.hip -- Q8_0-weight GEMV for gfx950.
//
// y[i] = sum_k dequant(W)[i][k] * x[k] (+ residual[i]).  Q8_0 blocks
// (runtime/zig/src/doe_wgsl/csl_spec.zig:122-152, the `q8_0` quant format of
// emit_csl_host.zig:62) hold 32 weights in 34 bytes: an f16 scale d, then 32
// int8 quants q; weight = d * q.  Weights are row-wise: each row is
// nb = ceil(k / 32) blocks (the tail block zero padded), so a row is nb * 34
// bytes and blocks are only 2-byte aligned.
//
// Decomposition: a workgroup of four waves first issues the loads of its first
// blocks, then stages x into LDS as 36-float rows per block (32 values + 4 of
// padding: lanes on consecutive blocks hit distinct banks; 16-byte loads when
// x is 16-byte aligned) together with the per-block sums sx[b], reduced in
// registers on the way.  A wave owns groups of R consecutive rows; the R * nb
// (row, block) units of a group are spread over its lanes (unit u = lane +
// 64 t), so short rows still fill the wave.  A unit is three buffer loads
// (16 + 16 + 4 bytes from the block's dword-aligned start: no 64-bit address
// registers, and bytes past the matrix read as zero), one v_perm per quant
// dword to undo the 2-byte misalignment, and 32 FMAs of u = q + 128 (the
// sign bit flipped, so each byte converts with one v_cvt_f32_ubyte) against x:
// block dot = d * (sum u * x - 128 * sx[b]).  The next unit's loads are issued
// before the current unit is computed.  Bound: HBM (34 bytes per 32 weights).
#include "common.h"

#include <string.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;               // waves per workgroup
constexpr int kXStride = 36;            // floats per staged x block (32 + pad)
constexpr int kMaxBlocks = 1024;        // k <= 32768: 1024 * 148 bytes of LDS
constexpr uint32_t kOutOfRange = 0x80000000u;  // buffer offset that reads zero

struct Blk {
    u32x4 a, b;
    uint32_t c;
};

__device__ __forceinline__ Blk load_blk(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    const uint32_t al = off & ~3u;
    Blk r;
    r.a = __builtin_amdgcn_raw_buffer_load_b128(rs, al, 0, 0);
    r.b = __builtin_amdgcn_raw_buffer_load_b128(rs, al + 16, 0, 0);
    r.c = __builtin_amdgcn_raw_buffer_load_b32(rs, al + 32, 0, 0);
    return r;
}

// d * sum_j q_j * x_j for the block whose 34 bytes start at byte (off & 3)
// of the loaded dwords; xb = the block's staged x, sxb = their sum.
__device__ __forceinline__ float blk_dot(const Blk &bk, uint32_t off, const float *xb, float sxb) {
    const uint32_t dw[9] = {bk.a.x, bk.a.y, bk.a.z, bk.a.w, bk.b.x, bk.b.y, bk.b.z, bk.b.w, bk.c};
    const uint32_t sh = (off & 2u) << 3;                    // 0 or 16
    const uint32_t sel = sh ? 0x07060504u : 0x05040302u;   // quant bytes at 4 or 2
    const float d = doe_half_bits_to_float(__builtin_amdgcn_ubfe(dw[0], sh, 16));
    const float4 *x4 = reinterpret_cast<const float4 *>(xb);
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t u = __builtin_amdgcn_perm(dw[j + 1], dw[j], sel) ^ 0x80808080u;
        const float4 xv = x4[j];
        s0 = fmaf((float)(u & 0xffu), xv.x, s0);
        s1 = fmaf((float)((u >> 8) & 0xffu), xv.y, s1);
        s0 = fmaf((float)((u >> 16) & 0xffu), xv.z, s0);
        s1 = fmaf((float)(u >> 24), xv.w, s1);
    }
    return d * fmaf(-128.0f, sxb, s0 + s1);
}

// The activation as split-attention partials (doe_attn_decode_partials):
// x[h * D + d] = sum_s o[h][s][d] 2^(m_s - M) / sum_s l_s 2^(m_s - M),
// M = max_s m_s, with o [heads][S][D] then (m, l) [heads][S][2].
constexpr int kAttnMaxSplits = 8;

struct Q8Attn {
    const float *o;   // nullptr: x is a plain f32 vector
    const float *ml;
    int splits, head_dim;
};

__device__ __forceinline__ float4 attn_combine4(const Q8Attn &at, int e) {
    const int S = at.splits, D = at.head_dim;
    const int h = e / D, d = e - h * D;  // e % 4 == 0 and D % 4 == 0: one head
    float2 ml[kAttnMaxSplits];
    float M = -INFINITY;
#pragma unroll
    for (int sp = 0; sp < kAttnMaxSplits; ++sp) {
        if (sp < S) {
            ml[sp] = *reinterpret_cast<const float2 *>(at.ml + ((size_t)h * S + sp) * 2);
            M = fmaxf(M, ml[sp].x);
        }
    }
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float L = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
        for (int sp = 0; sp < kAttnMaxSplits; ++sp) {
            if (sp < S) {
                const float f = exp2f(ml[sp].x - M);
                const float4 o = *reinterpret_cast<const float4 *>(at.o + ((size_t)h * S + sp) * D + d);
                L = fmaf(ml[sp].y, f, L);
                acc.x = fmaf(o.x, f, acc.x);
                acc.y = fmaf(o.y, f, acc.y);
                acc.z = fmaf(o.z, f, acc.z);
                acc.w = fmaf(o.w, f, acc.w);
            }
        }
    }
    const float rl = L > 0.0f ? 1.0f / L : 0.0f;
    return make_float4(acc.x * rl, acc.y * rl, acc.z * rl, acc.w * rl);
}

// Epilogues over row pairs (2i, 2i + 1) of a wave group (R even): the GeGLU of
// interleaved gate/up rows, y[i] = gelu_tanh(dot_2i) * dot_2i+1
// (gelu_gated.wgsl:1-14), or RoPE + the K/V cache write of a fused q/k/v
// projection whose q/k rows are interleaved rotation pairs (doe_rope_kv_pair).
struct Q8Epi {
    int gated, rope_kv;
    DoeRopeKv rk;
};

template <int R, int D>
__global__ __launch_bounds__(kWaves * 64) void q8_0_gemv_kernel(
    const uint8_t *__restrict__ w, const float *__restrict__ x, float *y, const float *res, int n,
    int k, int nb, int q64, int r64, bool x_vec, const float *norm_w, float norm_eps, int norm_offset,
    Q8Attn at, Q8Epi ep) {
    static_assert(D == 1 || D == 2, "one or two units in flight ahead");
    extern __shared__ float lds[];
    float *xs = lds;                          // [nb][kXStride]
    float *sx = lds + (size_t)nb * kXStride;  // [nb]
    float *ss = sx + nb;                      // [kWaves] sums of squares (norm)
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int nwaves = gridDim.x * kWaves;
    const int ngroups = (n + R - 1) / R;
    const uint32_t rb = (uint32_t)nb * 34u;  // row bytes
    // first unit of every group: row lane / nb, block lane % nb; each round
    // moves a lane 64 units on: q64 rows and r64 blocks
    const int rl0 = lane / nb, b0 = lane - rl0 * nb;
    auto adv = [&](int &r, int &bb) {
        r += q64;
        bb += r64;
        if (bb >= nb) {
            bb -= nb;
            ++r;
        }
    };

    int g = wave, rows = 0, rounds = 0, lrl = 0, lb = 0;
    uint32_t s0 = 0;
    __amdgpu_buffer_rsrc_t rs;
    Blk c0, c1;
    uint32_t o0 = kOutOfRange, o1 = kOutOfRange;
    // group g's buffer and its first D units' loads (a wave without a group
    // reads out of range: zeros, no access)
    auto start_group = [&]() {
        const int gg = min(g, ngroups - 1);
        rows = min(R, n - gg * R);
        rounds = g < ngroups ? (rows * nb + 63) >> 6 : 0;
        const size_t base = (size_t)gg * R * rb;
        s0 = (uint32_t)(base & 3u);
        rs = __builtin_amdgcn_make_buffer_rsrc((void *)(w + base - s0), (short)0,
                                               (int)((s0 + (uint32_t)rows * rb + 3u) & ~3u), 0x00020000);
        lrl = rl0;
        lb = b0;
        o0 = (0 < rounds && lrl < rows) ? s0 + (uint32_t)lrl * rb + 34u * (uint32_t)lb : kOutOfRange;
        c0 = load_blk(rs, o0);
        adv(lrl, lb);
        if (D == 2) {
            o1 = (1 < rounds && lrl < rows) ? s0 + (uint32_t)lrl * rb + 34u * (uint32_t)lb : kOutOfRange;
            c1 = load_blk(rs, o1);
            adv(lrl, lb);
        }
    };
    start_group();  // issued before x is staged

    // x in 4-float pieces (piece i = elements 4i..4i+3 of block i / 8); the
    // eight lanes holding a block's pieces sum it with three shuffles.  With
    // an RMSNorm, x * w' is staged (w' = w or 1 + w) and the row sums are
    // scaled by 1 / sqrt(mean(x^2) + eps) at the end: W (r x w') = r W (x w').
    float sq = 0.0f;
    for (int i0 = 0; i0 < nb * 8; i0 += kWaves * 64) {
        const int i = i0 + threadIdx.x;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (i < nb * 8) {
            const int e = 4 * i;
            if (at.o) {
                if (e < k) v = attn_combine4(at, e);  // k % 4 == 0 in this form
            } else if (x_vec && e + 3 < k) {
                v = *reinterpret_cast<const float4 *>(x + e);
            } else {
                if (e < k) v.x = x[e];
                if (e + 1 < k) v.y = x[e + 1];
                if (e + 2 < k) v.z = x[e + 2];
                if (e + 3 < k) v.w = x[e + 3];
            }
            if (norm_w) {
                sq += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
                const float o = norm_offset ? 1.0f : 0.0f;
                v.x *= o + (e < k ? norm_w[e] : 0.0f);
                v.y *= o + (e + 1 < k ? norm_w[e + 1] : 0.0f);
                v.z *= o + (e + 2 < k ? norm_w[e + 2] : 0.0f);
                v.w *= o + (e + 3 < k ? norm_w[e + 3] : 0.0f);
            }
            *reinterpret_cast<float4 *>(xs + (i >> 3) * kXStride + (i & 7) * 4) = v;
        }
        float s = (v.x + v.y) + (v.z + v.w);
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        s += __shfl_xor(s, 4, 64);
        if (i < nb * 8 && (i & 7) == 0) sx[i >> 3] = s;
    }
    if (norm_w) {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) sq += __shfl_xor(sq, o, 64);
        if (lane == 0) ss[threadIdx.x >> 6] = sq;
    }
    __syncthreads();
    float rms_inv = 1.0f;
    if (norm_w) {
        float t = 0.0f;
#pragma unroll
        for (int j = 0; j < kWaves; ++j) t += ss[j];
        rms_inv = 1.0f / sqrtf(t / (float)k + norm_eps);
    }

    for (; g < ngroups; g += nwaves) {
        if (g != wave) start_group();
        int rl = rl0, b = b0;
        float acc[R];
#pragma unroll
        for (int j = 0; j < R; ++j) acc[j] = 0.0f;
        for (int t = 0; t < rounds; ++t) {
            const uint32_t on =
                (t + D < rounds && lrl < rows) ? s0 + (uint32_t)lrl * rb + 34u * (uint32_t)lb : kOutOfRange;
            const Blk cn = load_blk(rs, on);
            adv(lrl, lb);
            const float v = blk_dot(c0, o0, xs + b * kXStride, sx[b]);
#pragma unroll
            for (int j = 0; j < R; ++j) acc[j] += (rl == j) ? v : 0.0f;
            adv(rl, b);
            if (D == 2) {
                c0 = c1;
                o0 = o1;
                c1 = cn;
                o1 = on;
            } else {
                c0 = cn;
                o0 = on;
            }
        }
        float sum[R];
#pragma unroll
        for (int j = 0; j < R; ++j) {
            float s = acc[j];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
            sum[j] = s;
        }
        if (ep.gated || ep.rope_kv) {  // wave-uniform; R is even and so is n
#pragma unroll
            for (int j = 0; j + 1 < R; j += 2) {
                if (lane == 0 && j < rows) {
                    const int row = g * R + j;
                    const float s0 = rms_inv * sum[j], s1 = rms_inv * sum[j + 1];
                    if (ep.gated) y[row >> 1] = doe_gelu_tanh_clamped(s0) * s1;
                    else doe_rope_kv_pair(ep.rk, row, s0, s1, y);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < R; ++j) {
                if (lane == 0 && j < rows) {
                    const int row = g * R + j;
                    y[row] = res ? fmaf(rms_inv, sum[j], res[row]) : rms_inv * sum[j];
                }
            }
        }
    }
}

int g_num_cus = 0;

int g_tune_rows = 0;   // 0 = automatic, else 1, 2 or 4 rows per wave group
int g_tune_depth = 0;  // 0 = automatic, else 1 or 2 units in flight ahead

struct Q8Norm {
    const float *norm_w;  // nullptr: no RMSNorm of the activation
    float norm_eps;
    int norm_offset;
};

template <int R, int D>
int q8_0_launch(const uint8_t *w, const float *x, float *y, const float *res, int n, int k, int nb,
                const Q8Norm &fz, const Q8Attn &at, const Q8Epi &ep, hipStream_t st) {
    static const hipError_t attr_rc = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&q8_0_gemv_kernel<R, D>),
        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxBlocks * (kXStride + 1) * 4 + kWaves * 4);
    DOE_HIP_CHECK(attr_rc);
    const long ngroups = (n + R - 1) / R;
    long blocks = (ngroups + kWaves - 1) / kWaves;
    const long cap = (long)g_num_cus * 8;
    if (blocks > cap) blocks = cap;
    const size_t lds = (size_t)nb * (kXStride + 1) * 4 + kWaves * 4;
    hipLaunchKernelGGL((q8_0_gemv_kernel<R, D>), dim3((unsigned)blocks), dim3(kWaves * 64), lds, st,
                       w, x, y, res, n, k, nb, 64 / nb, 64 % nb, ((uintptr_t)x & 15) == 0, fz.norm_w,
                       fz.norm_eps, fz.norm_offset, at, ep);
    DOE_LAUNCH_CHECK("q8_0_gemv_kernel");
    return DOE_OK;
}

template <int R>
int q8_0_launch_depth(const uint8_t *w, const float *x, float *y, const float *res, int n, int k,
                      int nb, const Q8Norm &fz, const Q8Attn &at, const Q8Epi &ep, hipStream_t st) {
    if (g_tune_depth == 2) return q8_0_launch<R, 2>(w, x, y, res, n, k, nb, fz, at, ep, st);
    return q8_0_launch<R, 1>(w, x, y, res, n, k, nb, fz, at, ep, st);
}

}  // namespace

namespace {

int q8_0_gemv_impl(const void *weight_q8_0, const float *activation, float *output, int64_t n,
                   int64_t k, const float *residual, const Q8Norm &fz, doe_stream_t stream,
                   const Q8Attn &at = Q8Attn{nullptr, nullptr, 0, 0}, const Q8Epi &ep = Q8Epi{}) {
    int rc = doe::require_init();
    if (rc) return rc;
    const hipStream_t st = (hipStream_t)stream;
    DOE_REQUIRE(n >= 0 && k >= 0 && n <= 0x7fffffff, DOE_E_INVALID, "bad q8_0_gemv shape");
    if (n == 0) return DOE_OK;
    DOE_REQUIRE(output, DOE_E_INVALID, "null output");
    const bool paired = ep.gated || ep.rope_kv;
    DOE_REQUIRE(!paired || (n % 2 == 0 && k > 0 && !residual), DOE_E_INVALID,
                "the GeGLU and RoPE epilogues need an even row count, k > 0 and no residual");
    if (k == 0) {  // empty reductions: the residual, or zeros
        if (!residual) return doe::fill_bytes_async(output, 0, (size_t)n * 4, st);
        if (residual != output)
            DOE_HIP_CHECK(hipMemcpyAsync(output, residual, (size_t)n * 4, hipMemcpyDeviceToDevice, st));
        return DOE_OK;
    }
    DOE_REQUIRE(weight_q8_0 && (activation || at.o), DOE_E_INVALID, "null pointer");
    // every workgroup stages the whole activation while others already write
    // output rows: only the residual may alias the output
    DOE_REQUIRE(activation != output && fz.norm_w != output && (!at.o || (at.o != output && at.ml != output)),
                DOE_E_INVALID, "the activation and norm weight must not alias the output (only the residual may)");
    const int64_t nb = (k + 31) / 32;
    DOE_REQUIRE(nb <= kMaxBlocks, DOE_E_UNSUPPORTED,
                "q8_0_gemv needs k <= %d (got %lld)", kMaxBlocks * 32, (long long)k);
    DOE_REQUIRE(((uintptr_t)weight_q8_0 & 3) == 0, DOE_E_INVALID, "Q8_0 weights must be 4-byte aligned");
    DOE_REQUIRE(((uintptr_t)activation & 3) == 0 && ((uintptr_t)output & 3) == 0 &&
                    ((uintptr_t)residual & 3) == 0 && ((uintptr_t)fz.norm_w & 3) == 0,
                DOE_E_INVALID, "activation, output, residual and norm weight must be 4-byte aligned");
    if (g_num_cus == 0) {
        int dev = 0, cus = 0;
        DOE_HIP_CHECK(hipGetDevice(&dev));
        DOE_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        g_num_cus = cus > 0 ? cus : 256;
    }
    const uint8_t *w = (const uint8_t *)weight_q8_0;
    // rows per wave group: the fewest that give a wave two full rounds of
    // units (a partly filled last round idles lanes) while two workgroups per
    // CU remain, more where the persistent grid is full anyway (fewer groups,
    // same occupancy)
    int r = g_tune_rows;
    if (r == 0) {
        r = 1;
        while (r < 4 && (int64_t)r * nb < 128 &&
               (n + 2 * r - 1) / (2 * r) >= (int64_t)g_num_cus * 2 * kWaves)
            r *= 2;
        while (r < 4 && (n + r - 1) / r > (int64_t)g_num_cus * 8 * kWaves) r *= 2;
    }
    if (paired && r == 1) r = 2;  // a wave group holds whole row pairs
    if (r == 4)
        return q8_0_launch_depth<4>(w, activation, output, residual, (int)n, (int)k, (int)nb, fz, at, ep, st);
    if (r == 2)
        return q8_0_launch_depth<2>(w, activation, output, residual, (int)n, (int)k, (int)nb, fz, at, ep, st);
    return q8_0_launch_depth<1>(w, activation, output, residual, (int)n, (int)k, (int)nb, fz, at, ep, st);
}

}  // namespace

extern "C" int doe_q8_0_gemv(const void *weight_q8_0, const float *activation, float *output,
                             int64_t n, int64_t k, const float *residual, doe_stream_t stream) {
    return q8_0_gemv_impl(weight_q8_0, activation, output, n, k, residual, Q8Norm{nullptr, 0.0f, 0},
                          stream);
}

extern "C" int doe_q8_0_gemv_norm(const void *weight_q8_0, const float *activation, float *output,
                                  int64_t n, int64_t k, const float *norm_weight, float norm_eps,
                                  int norm_weight_offset, const float *residual, doe_stream_t stream) {
    DOE_REQUIRE(norm_weight, DOE_E_INVALID, "null norm weight");
    return q8_0_gemv_impl(weight_q8_0, activation, output, n, k, residual,
                          Q8Norm{norm_weight, norm_eps, norm_weight_offset ? 1 : 0}, stream);
}

extern "C" int doe_q8_0_gemv_attn_out(const void *weight_q8_0, const float *attn_partials, int64_t splits,
                                      int64_t num_heads, int64_t head_dim, float *output, int64_t n,
                                      const float *residual, doe_stream_t stream) {
    DOE_REQUIRE(attn_partials, DOE_E_INVALID, "null partials");
    DOE_REQUIRE(splits >= 1 && splits <= kAttnMaxSplits, DOE_E_UNSUPPORTED,
                "attention combine prologue supports 1..%d splits (got %lld)", kAttnMaxSplits, (long long)splits);
    DOE_REQUIRE(num_heads > 0 && head_dim > 0 && head_dim % 4 == 0 && num_heads * head_dim <= 0x7fffffff,
                DOE_E_INVALID, "bad head shape");
    DOE_REQUIRE(((uintptr_t)attn_partials & 15) == 0, DOE_E_INVALID, "partials must be 16-byte aligned");
    const Q8Attn at{attn_partials, attn_partials + num_heads * splits * head_dim, (int)splits, (int)head_dim};
    return q8_0_gemv_impl(weight_q8_0, nullptr, output, n, num_heads * head_dim, residual,
                          Q8Norm{nullptr, 0.0f, 0}, stream, at);
}

extern "C" int doe_q8_0_gemv_fused(const void *weight_q8_0, const float *activation, float *output, int64_t n,
                                   int64_t k, const float *norm_weight, float norm_eps, int norm_weight_offset,
                                   const float *residual, int gated, doe_stream_t stream) {
    DOE_REQUIRE(!gated || !residual, DOE_E_INVALID, "gated and residual are exclusive");
    Q8Epi ep{};
    ep.gated = gated ? 1 : 0;
    return q8_0_gemv_impl(weight_q8_0, activation, output, n, k, residual,
                          Q8Norm{norm_weight, norm_eps, norm_weight_offset ? 1 : 0}, stream,
                          Q8Attn{nullptr, nullptr, 0, 0}, ep);
}

extern "C" int doe_q8_0_gemv_qkv_rope_kv(const void *weight_q8_0, const float *activation, float *output,
                                         int64_t hidden, const float *norm_weight, float norm_eps,
                                         int norm_weight_offset, int64_t num_heads, int64_t num_kv_heads,
                                         int64_t head_dim, const float *freq_cis, const int32_t *position_dev,
                                         uint16_t *key_cache, uint16_t *val_cache, int64_t max_seq_len,
                                         doe_stream_t stream) {
    DOE_REQUIRE(num_heads > 0 && num_kv_heads >= 0 && head_dim > 0 && (head_dim % 2) == 0 && max_seq_len > 0 &&
                    (num_heads + 2 * num_kv_heads) * head_dim <= 0x7fffffff,
                DOE_E_INVALID, "bad qkv shape");
    DOE_REQUIRE(freq_cis && position_dev && (num_kv_heads == 0 || (key_cache && val_cache)), DOE_E_INVALID,
                "null pointer");
    Q8Epi ep{};
    ep.rope_kv = 1;
    ep.rk = DoeRopeKv{freq_cis, position_dev, (_Float16 *)key_cache, (_Float16 *)val_cache,
                      (int)(num_heads * head_dim), (int)(num_kv_heads * head_dim), (int)head_dim, (int)max_seq_len};
    const int64_t n = (num_heads + 2 * num_kv_heads) * head_dim;
    return q8_0_gemv_impl(weight_q8_0, activation, output, n, hidden, nullptr,
                          Q8Norm{norm_weight, norm_eps, norm_weight_offset ? 1 : 0}, stream,
                          Q8Attn{nullptr, nullptr, 0, 0}, ep);
}

namespace doe {

int q8_0_set_tune(const char *key, int v) {
    if (!strcmp(key, "q8_0_gemv.rows")) {
        DOE_REQUIRE(v == 0 || v == 1 || v == 2 || v == 4, DOE_E_INVALID, "q8_0_gemv.rows is 0, 1, 2 or 4");
        g_tune_rows = v;
    } else {
        DOE_REQUIRE(v >= 0 && v <= 2, DOE_E_INVALID, "q8_0_gemv.depth is 0, 1 or 2");
        g_tune_depth = v;
    }
    return DOE_OK;
}

}  // namespace doe
