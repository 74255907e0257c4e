// attn_prefill.hip -- causal GQA prefill attention (flash form) on gfx950 matrix cores.
//
// out[i][h][:] = softmax_j(q[i][h] . k[kvh][j] * scale) v[kvh][j], kvh = h / (Hq/Hkv),
// keys j <= start_pos + i when causal -- the reference's tiled attention
// (attention_head256_f16kv.wgsl:72-267 with is_causal, query blocks; CPU
// tiled online softmax run_csl_webgpu_emulator.mjs:646-720).  q is bf16
// [q_len][Hq][128], k/v bf16 [Hkv][kv_stride][128] (the cache layout
// [kv_head][pos][dim]), out f32 or bf16 [q_len][Hq][128].
//
// One workgroup = 128 queries of one head (four waves of 32), keys in blocks
// of 64 staged in LDS (double-buffered, the next block's loads in flight).
// Per wave and key block:
//   * S^T = K . Q^T on v_mfma_f32_32x32x16_bf16 (bf16 inputs are exact, f32
//     accumulate).  The transposed product puts one query per lane column, so
//     the online softmax needs no cross-lane reductions except one exchange
//     between the two lane halves that hold the same query.
//   * P = exp2(S*scale*log2e - m) in f32, rounded to f16, and O^T += V^T . P^T
//     on v_mfma_f32_32x32x16_f16: P's registers are used in place as the B
//     operand (the key order of the product follows the MFMA's D layout; V^T is
//     read in the same order).  V is staged transposed in LDS and converted
//     bf16 -> f16 on the way (exact for |v| in [2^-14, 65504]); f16 P keeps
//     the output near 1e-4 rel-L2, where a bf16 P would sit at ~1e-3.
// Query blocks are dispatched heavy and light in complementary halves so the
// two workgroups resident on a CU carry about the same number of key blocks.
#include "common.h"

#include <math.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kD = 128, kBQ = 128, kBKV = 64;
constexpr int kKRow = kD + 8;     // bf16 per K row in LDS (272 B: b128 reads conflict-free)
constexpr int kVRow = kBKV + 12;  // f16 per V^T row in LDS (152 B: b64 reads conflict-free)

struct PrefillArgs {
    const uint16_t *q, *k, *v;
    void *out;
    int hq, hkv, q_len, kv_len, kv_stride, start_pos, causal, out_bf16, nqb;
    float scale_log2;  // softmax scale * log2(e)
};

__device__ __forceinline__ uint32_t bf16pair_to_f16pair(uint32_t w) {
    const float lo = __uint_as_float(w << 16), hi = __uint_as_float(w & 0xffff0000u);
    const _Float16 a = (_Float16)lo, b = (_Float16)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_prefill_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kBKV * kKRow];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[2][kD * kVRow];

    const int h = blockIdx.x % a.hq;
    const int slot = blockIdx.x / a.hq;
    const int half = (a.nqb + 1) / 2;
    const int qb = slot < half ? a.nqb - 1 - slot : slot - half;
    const int kvh = h / (a.hq / a.hkv);
    const int q0 = qb * kBQ;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 31, lg = lane >> 5;
    const int qi = q0 + wave * 32 + lr;  // this lane's query (column of S^T)
    const int qrow = min(qi, a.q_len - 1);

    // Q^T operand fragments: Q[qi][h][16 s + 8 lg .. + 8]
    bf16x8 qf[8];
    {
        const uint16_t *qp = a.q + ((size_t)qrow * a.hq + h) * kD + 8 * lg;
#pragma unroll
        for (int s = 0; s < 8; ++s) qf[s] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(qp + 16 * s));
    }

    const int q_last = min(q0 + kBQ, a.q_len) - 1;
    const int kv_end = a.causal ? min(a.kv_len, a.start_pos + q_last + 1) : a.kv_len;
    const int nkb = (kv_end + kBKV - 1) / kBKV;
    // keys this lane's query may see: [0, limit)
    const int limit = qi < a.q_len ? (a.causal ? min(a.kv_len, a.start_pos + qi + 1) : a.kv_len) : kv_end;

    const uint16_t *kbase = a.k + (size_t)kvh * a.kv_stride * kD;
    const uint16_t *vbase = a.v + (size_t)kvh * a.kv_stride * kD;
    // K staging: granule gi = tid + 256 i -> key gi >> 4, column (gi & 15) * 8
    // V staging: keys 4 (tid >> 4) .. + 3, dims 8 (tid & 15) .. + 7
    const int vkg = tid >> 4, vdg = tid & 15;
    u32x4 rk[4], rv[4];
#define DOE_PF_LOAD(KB)                                                                              \
    do {                                                                                             \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                              \
            const int gi = tid + 256 * i;                                                            \
            const int key = min((KB) * kBKV + (gi >> 4), a.kv_len - 1);                              \
            rk[i] = *reinterpret_cast<const u32x4 *>(kbase + (size_t)key * kD + (gi & 15) * 8);      \
            const int vkey = min((KB) * kBKV + 4 * vkg + i, a.kv_len - 1);                           \
            rv[i] = *reinterpret_cast<const u32x4 *>(vbase + (size_t)vkey * kD + 8 * vdg);           \
        }                                                                                            \
    } while (0)
#define DOE_PF_STORE(BUF)                                                                            \
    do {                                                                                             \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                              \
            const int gi = tid + 256 * i;                                                            \
            *reinterpret_cast<u32x4 *>(&Ks[BUF][(gi >> 4) * kKRow + (gi & 15) * 8]) = rk[i];         \
        }                                                                                            \
        /* f16 pairs (d 2e, d 2e+1) of each of the 4 keys, then transpose to V^T rows */            \
        uint32_t hv[4][4];                                                                           \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                              \
            hv[i][0] = bf16pair_to_f16pair(rv[i].x);                                                 \
            hv[i][1] = bf16pair_to_f16pair(rv[i].y);                                                 \
            hv[i][2] = bf16pair_to_f16pair(rv[i].z);                                                 \
            hv[i][3] = bf16pair_to_f16pair(rv[i].w);                                                 \
        }                                                                                            \
        _Pragma("unroll") for (int e = 0; e < 4; ++e) {                                              \
            /* dims 2e (low halves) and 2e+1 (high halves) over keys 0..3 */                         \
            const u32x2 lo = {__builtin_amdgcn_perm(hv[1][e], hv[0][e], 0x05040100u),                \
                              __builtin_amdgcn_perm(hv[3][e], hv[2][e], 0x05040100u)};               \
            const u32x2 hi = {__builtin_amdgcn_perm(hv[1][e], hv[0][e], 0x07060302u),                \
                              __builtin_amdgcn_perm(hv[3][e], hv[2][e], 0x07060302u)};               \
            *reinterpret_cast<u32x2 *>(&Vt[BUF][(8 * vdg + 2 * e) * kVRow + 4 * vkg]) = lo;          \
            *reinterpret_cast<u32x2 *>(&Vt[BUF][(8 * vdg + 2 * e + 1) * kVRow + 4 * vkg]) = hi;      \
        }                                                                                            \
    } while (0)

    float16v o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
    float m_i = -INFINITY, l_i = 0.0f;

    if (nkb > 0) {
        DOE_PF_LOAD(0);
        DOE_PF_STORE(0);
    }
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
        const int buf = kb & 1;
        if (kb + 1 < nkb) DOE_PF_LOAD(kb + 1);
        // S^T for keys 64 kb + 32 kb2 + [0, 32): D[i] = key (i%4) + 8(i/4) + 4 lg, query lr
        float16v st[2];
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
            for (int r = 0; r < 16; ++r) st[kb2][r] = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const bf16x8 kf = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4 *>(&Ks[buf][(32 * kb2 + lr) * kKRow + 16 * s + 8 * lg]));
                st[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], st[kb2], 0, 0, 0);
            }
        }
        // online softmax (base 2), one query per lane column
        float bmax = -INFINITY;
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kb * kBKV + 32 * kb2 + (r & 3) + 8 * (r >> 2) + 4 * lg;
                const float x = key < limit ? st[kb2][r] * a.scale_log2 : -INFINITY;
                st[kb2][r] = x;
                bmax = fmaxf(bmax, x);
            }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
        const float m_new = fmaxf(m_i, bmax);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_i - m_use);
        m_i = m_new;
        float psum = 0.0f;
        half8 pf[4];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = __builtin_amdgcn_exp2f(st[s4 >> 1][8 * (s4 & 1) + j] - m_use);
                psum += p;
                pf[s4][j] = (_Float16)p;
            }
        l_i = l_i * alpha + psum;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
        // O^T[d][q] += V^T[d][keys] . P^T[keys][q]; slot 8 lg + j of slice s4 is key
        // 32 (s4/2) + 16 (s4%2) + 4 lg + (j%4) + 8 (j/4) -- the D layout of S^T
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            const int key0 = 32 * (s4 >> 1) + 16 * (s4 & 1) + 4 * lg;
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const _Float16 *vr = &Vt[buf][(32 * db + lr) * kVRow + key0];
                const u32x2 v0 = *reinterpret_cast<const u32x2 *>(vr);
                const u32x2 v1 = *reinterpret_cast<const u32x2 *>(vr + 8);
                const half8 vf = __builtin_bit_cast(half8, u32x4{v0.x, v0.y, v1.x, v1.y});
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[s4], o[db], 0, 0, 0);
            }
        }
        if (kb + 1 < nkb) DOE_PF_STORE(buf ^ 1);
        __syncthreads();
    }
#undef DOE_PF_LOAD
#undef DOE_PF_STORE

    if (qi >= a.q_len) return;
    const float l_tot = l_i + __shfl_xor(l_i, 32, 64);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    const size_t obase = ((size_t)qi * a.hq + h) * kD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int d0 = 32 * db + 8 * r4 + 4 * lg;
            const float v0 = o[db][4 * r4] * inv, v1 = o[db][4 * r4 + 1] * inv;
            const float v2 = o[db][4 * r4 + 2] * inv, v3 = o[db][4 * r4 + 3] * inv;
            if (a.out_bf16) {
                const u32x2 w = {(uint32_t)f32_to_bf16_rne(v0) | ((uint32_t)f32_to_bf16_rne(v1) << 16),
                                 (uint32_t)f32_to_bf16_rne(v2) | ((uint32_t)f32_to_bf16_rne(v3) << 16)};
                *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(a.out) + obase + d0) = w;
            } else {
                *reinterpret_cast<float4 *>(reinterpret_cast<float *>(a.out) + obase + d0) = make_float4(v0, v1, v2, v3);
            }
        }
}

}  // namespace

extern "C" {

int doe_attn_prefill(const uint16_t *q, const uint16_t *k, const uint16_t *v, void *out, int out_bf16,
                     int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t q_len,
                     int64_t kv_len, int64_t kv_stride, int64_t start_pos, float scale, int causal,
                     doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(num_heads > 0 && num_kv_heads > 0 && q_len >= 0 && kv_len >= 0 && start_pos >= 0,
                DOE_E_INVALID, "bad prefill attention shape");
    DOE_REQUIRE(num_heads % num_kv_heads == 0, DOE_E_INVALID,
                "num_heads %lld is not a multiple of num_kv_heads %lld", (long long)num_heads,
                (long long)num_kv_heads);
    DOE_REQUIRE(head_dim == kD, DOE_E_UNSUPPORTED, "prefill attention supports head_dim 128 (got %lld)",
                (long long)head_dim);
    DOE_REQUIRE(kv_stride >= kv_len, DOE_E_INVALID, "kv_stride %lld < kv_len %lld", (long long)kv_stride,
                (long long)kv_len);
    DOE_REQUIRE(num_heads <= 4096 && q_len <= (1 << 24) && kv_stride <= (1 << 24) &&
                    num_kv_heads * kv_stride * kD <= ((int64_t)1 << 40),
                DOE_E_UNSUPPORTED, "prefill attention shape too large");
    if (q_len == 0) return DOE_OK;
    DOE_REQUIRE(q && out && (kv_len == 0 || (k && v)), DOE_E_INVALID, "null pointer");
    DOE_REQUIRE((((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15) == 0, DOE_E_INVALID,
                "q, k, v and out must be 16-byte aligned");
    PrefillArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.hq = (int)num_heads;
    a.hkv = (int)num_kv_heads;
    a.q_len = (int)q_len;
    a.kv_len = (int)kv_len;
    a.kv_stride = (int)kv_stride;
    a.start_pos = (int)start_pos;
    a.causal = causal ? 1 : 0;
    a.out_bf16 = out_bf16 ? 1 : 0;
    a.nqb = (int)((q_len + kBQ - 1) / kBQ);
    a.scale_log2 = scale * 1.4426950408889634f;
    hipStream_t st = (hipStream_t)stream;
    if (kv_len == 0) {
        // no keys: the empty softmax contributes nothing (zero output)
        const size_t bytes = (size_t)q_len * num_heads * kD * (out_bf16 ? 2 : 4);
        DOE_HIP_CHECK(hipMemsetAsync(out, 0, bytes, st));
        return DOE_OK;
    }
    const int64_t blocks = (int64_t)a.nqb * a.hq;
    DOE_REQUIRE(blocks <= 0x7fffffff, DOE_E_UNSUPPORTED, "too many blocks");
    hipLaunchKernelGGL(attn_prefill_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a);
    DOE_LAUNCH_CHECK("attn_prefill_kernel");
    return DOE_OK;
}

}  // extern "C"
