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
//   * P = exp2(S*scale*log2e - m) in f32 (one fma and one exp per score),
//     rounded to f16, and O^T += V^T . P^T on v_mfma_f32_32x32x16_f16: P's
//     registers are used in place as the B operand (the key order of the
//     product follows the MFMA's D layout; V^T is read in the same order).
//     The row sum l adds the same f16 P values (v_dot2_f32_f16).
//   * The running max m is raised (and O, l rescaled) only when some query's
//     block max exceeds it by more than 2^8: P stays <= 256, well inside f16,
//     and the O rescale runs on a few blocks instead of every block.
//   * The causal mask is evaluated only on the blocks that cross the
//     diagonal (or the end of the keys); blocks every query sees fully skip it.
// V is converted once per call by a pre-pass into an f16 V^T copy [Hkv][128]
// [keys] (exact for |v| in [2^-14, 65504]; f16 P keeps the output near 1e-4
// rel-L2, where a bf16 P would sit at ~1e-3), so the main loop copies V^T
// tiles straight into LDS.
// Query blocks are dispatched heavy and light in complementary halves so the
// two workgroups resident on a CU carry about the same number of key blocks.
#include "common.h"

#include <math.h>
#include <mutex>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kD = 128, kBQ = 128, kBKV = 64;
constexpr int kKRow = kD + 8;    // bf16 per K row in LDS (272 B: b128 reads conflict-free)
constexpr int kVRow = kBKV + 4;  // f16 per V^T row in LDS (136 B = 34 dwords: 16 lanes' b64 reads hit 32 distinct banks)
constexpr float kLazy = 8.0f;    // the running max is raised only past m + 8 (P <= 2^8)

struct PrefillArgs {
    const uint16_t *q, *k;
    const _Float16 *vt;  // f16 V^T [hkv][kD][kv_pad], keys >= kv_len zero
    void *out;
    int hq, hkv, q_len, kv_len, kv_stride, kv_pad, start_pos, causal, out_bf16, nqb;
    float scale_log2;  // softmax scale * log2(e)
};

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

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

// Pre-pass: V bf16 [hkv][kv_stride][128] -> f16 V^T [hkv][128][kv_pad] (keys
// past kv_len zero); one workgroup per 64 keys of one KV head, transposed
// through LDS.
__global__ __launch_bounds__(256) void v_to_f16t_kernel(const uint16_t *__restrict__ v, _Float16 *__restrict__ vt,
                                                        int kv_len, int kv_stride, int kv_pad) {
    __shared__ _Float16 tile[kBKV][kD + 2];  // [key][dim], odd dword stride
    const int kvh = blockIdx.y, key0 = blockIdx.x * kBKV, tid = threadIdx.x;
    // the four loads go out together (a key past kv_len reads a clamped key
    // and is zeroed after: no branch, so no load waits for the one before)
    u32x4 wl[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int gi = tid + 256 * i, kl = gi >> 4, d0 = (gi & 15) * 8;
        const int key = max(min(key0 + kl, kv_len - 1), 0);
        wl[i] = *reinterpret_cast<const u32x4 *>(v + ((size_t)kvh * kv_stride + key) * kD + d0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int gi = tid + 256 * i, kl = gi >> 4, d0 = (gi & 15) * 8;
        const uint32_t keep = key0 + kl < kv_len ? 0xffffffffu : 0u;  // (an and: the load is used either way)
        const u32x4 w = wl[i] & keep;
        const uint32_t p[4] = {bf16pair_to_f16pair(w.x), bf16pair_to_f16pair(w.y), bf16pair_to_f16pair(w.z),
                               bf16pair_to_f16pair(w.w)};
#pragma unroll
        for (int e = 0; e < 4; ++e) *reinterpret_cast<uint32_t *>(&tile[kl][d0 + 2 * e]) = p[e];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int gi = tid + 256 * i, d = gi >> 3, k0 = (gi & 7) * 8;
        half8 r;
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = tile[k0 + j][d];
        *reinterpret_cast<half8 *>(vt + ((size_t)kvh * kD + d) * kv_pad + key0 + k0) = r;
    }
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

    // K and V^T of this KV head as buffers: per-lane offsets fixed for the whole
    // loop, the block offset a scalar; keys past kv_len read as zero (masked)
    const __amdgpu_buffer_rsrc_t krsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.k + (size_t)kvh * a.kv_stride * kD), (short)0, a.kv_len * (kD * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.vt + (size_t)kvh * kD * a.kv_pad), (short)0, a.kv_pad * (kD * 2), 0x00020000);
    // K staging: granule gi = tid + 256 i -> key gi >> 4, column (gi & 15) * 8
    // V^T staging: dim tid >> 1, keys 32 (tid & 1) + 8 i .. + 7 of the block
    const int vd = tid >> 1, vh = tid & 1;
    const uint32_t k_voff = (uint32_t)((tid >> 4) * kD + (tid & 15) * 8) * 2u;  // + 16 keys per i
    const uint32_t v_voff = (uint32_t)(vd * a.kv_pad + 32 * vh) * 2u;           // + 8 keys per i
    // K runs one block ahead of V: in iteration kb, Ks[(kb + 1) & 1] holds
    // K(kb + 1) (the next block's scores are computed under this block's
    // softmax) and Vt[kb & 1] holds V(kb); K(kb + 2) and V(kb + 1) are loaded
    // during the iteration and written to the buffers freed by the previous
    // iteration's barrier.  Out-of-range block indices are clamped: their
    // loads stay inside the buffers and their results are never used.
    u32x4 rk[4], rv[4];
#define DOE_PF_LOAD_K(KB)                                                                            \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) rk[i] = __builtin_amdgcn_raw_buffer_load_b128(     \
        krsrc, k_voff + (uint32_t)i * (16 * kD * 2), (KB) * (kBKV * kD * 2), 0)
#define DOE_PF_LOAD_V(KB)                                                                            \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) rv[i] = __builtin_amdgcn_raw_buffer_load_b128(     \
        vrsrc, v_voff + (uint32_t)i * 16u, (KB) * (kBKV * 2), 0)
#define DOE_PF_STORE_K(BUF)                                                                          \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                                  \
        const int gi = tid + 256 * i;                                                                \
        *reinterpret_cast<u32x4 *>(&Ks[BUF][(gi >> 4) * kKRow + (gi & 15) * 8]) = rk[i];             \
    }
#define DOE_PF_STORE_V(BUF)                                                                          \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                                  \
        /* rows are 8-byte aligned: two b64 stores */                                                \
        u32x2 *dst = reinterpret_cast<u32x2 *>(&Vt[BUF][vd * kVRow + 32 * vh + 8 * i]);              \
        dst[0] = u32x2{rv[i].x, rv[i].y};                                                            \
        dst[1] = u32x2{rv[i].z, rv[i].w};                                                            \
    }

    float16v o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
    float m_i = -INFINITY, l_i = 0.0f;
    if (nkb == 0) {
        // no visible keys (only for rows past q_len): nothing to accumulate
    } else {
    // blocks [0, nkb_full) hold only keys every query of the workgroup sees
    const int vis_all = a.causal ? min(a.kv_len, a.start_pos + q0 + 1) : a.kv_len;
    const int nkb_full = min(nkb, vis_all / kBKV);
    const half2v ones = {(_Float16)1.0f, (_Float16)1.0f};

    // S^T of the block in Ks[buf]: D[i] = key (i%4) + 8(i/4) + 4 lg of half kb2, query lr
    auto s_mfmas = [&](float16v (&st)[2], const int buf) __attribute__((always_inline)) {
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
    };
    // masks block kbb's scores (keys >= limit -> -inf) and returns their raw max
    // over the query's two lane halves (the scale is positive: max commutes)
    auto block_max = [&](float16v (&st)[2], const int kbb, const bool mask) __attribute__((always_inline)) {
        float bmax = -INFINITY;
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                if (mask) {
                    const int key = kbb * kBKV + 32 * kb2 + (r & 3) + 8 * (r >> 2) + 4 * lg;
                    if (key >= limit) st[kb2][r] = -INFINITY;
                }
                bmax = fmaxf(bmax, st[kb2][r]);
            }
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(bmax), __float_as_uint(bmax), false, false);
        return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    };

    DOE_PF_LOAD_K(0);
    DOE_PF_LOAD_V(0);
    DOE_PF_STORE_K(0);
    DOE_PF_STORE_V(0);
    DOE_PF_LOAD_K(min(1, nkb - 1));
    DOE_PF_STORE_K(1);
    __syncthreads();
    float16v sc[2];
    s_mfmas(sc, 0);
    float bmax_c = block_max(sc, 0, nkb_full == 0);
    __syncthreads();  // every wave has read K(0) before iteration 0 overwrites Ks[0]

    // iteration kb: sc holds block kb's scores, sn receives block kb + 1's
    auto iter = [&](const int kb, const bool mask_next, float16v(&sc)[2], float16v(&sn)[2]) __attribute__((always_inline)) {
        const int vb = kb & 1, kn = (kb + 1) & 1;
        DOE_PF_LOAD_K(min(kb + 2, nkb - 1));
        DOE_PF_LOAD_V(min(kb + 1, nkb - 1));
        // running max for block kb (raised only past m + 8: P <= 2^8)
        const float mb = bmax_c * a.scale_log2;
        if (__builtin_amdgcn_ballot_w64(mb > m_i + kLazy) != 0) {  // wave-uniform
            const float m_new = fmaxf(m_i, mb);
            const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_i - m_new);
            m_i = m_new;
            l_i *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
        }
        const float nm = m_i == -INFINITY ? 0.0f : -m_i;
        // The next block's scores under this block's softmax: MFMA i of S^T
        // (half i % 2, dims 16 (i / 2)) with the K fragment read four MFMAs
        // ahead and score pair i of this block turned into f16 P.  Each step is
        // its own scheduling region, so the exp2s stay between the MFMAs.
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
            for (int r = 0; r < 16; ++r) sn[kb2][r] = 0.0f;
        auto kfrag = [&](const int i) __attribute__((always_inline)) {
            return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(
                                                  &Ks[kn][(32 * (i & 1) + lr) * kKRow + 16 * (i >> 1) + 8 * lg]));
        };
        constexpr int kAhead = 4;  // fragment reads this many MFMAs ahead of their use
        bf16x8 kf[kAhead + 1];
#pragma unroll
        for (int i = 0; i < kAhead; ++i) kf[i] = kfrag(i);
        half8 pf[4];
        float psum = 0.0f;
        // score pair i: slice i / 4, slots 2 (i % 4), 2 (i % 4) + 1.  Its exp2s
        // are issued in step i and converted / summed in step i + 1, so no
        // instruction waits on a just-issued transcendental (the wave issues
        // in order: such a wait would hold back the next MFMA).
        float pp0 = 0.0f, pp1 = 0.0f;
        auto finish_pair = [&](const int i) __attribute__((always_inline)) {
            const int s4 = i >> 2, j = 2 * (i & 3);
            const half2v h = {(_Float16)pp0, (_Float16)pp1};
            psum = __builtin_amdgcn_fdot2(h, ones, psum, false);
            pf[s4][j] = h[0];
            pf[s4][j + 1] = h[1];
        };
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            sn[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[i % (kAhead + 1)], qf[i >> 1], sn[i & 1], 0, 0, 0);
            if (i + kAhead < 16) kf[(i + kAhead) % (kAhead + 1)] = kfrag(i + kAhead);
            const int s4 = i >> 2, j = 2 * (i & 3);
            const float p0 = __builtin_amdgcn_exp2f(fmaf(sc[s4 >> 1][8 * (s4 & 1) + j], a.scale_log2, nm));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(sc[s4 >> 1][8 * (s4 & 1) + j + 1], a.scale_log2, nm));
            if (i > 0) finish_pair(i - 1);
            pp0 = p0;
            pp1 = p1;
            __builtin_amdgcn_sched_barrier(0);
        }
        finish_pair(15);
        l_i += psum;
        // O^T[d][q] += V^T[d][keys] . P^T[keys][q] (slot 8 lg + j of slice s4 is key
        // 32 (s4/2) + 16 (s4%2) + 4 lg + (j%4) + 8 (j/4) -- the D layout of S^T),
        // MFMA i = (slice i / 4, dims 32 (i % 4)) with its V^T fragment read four
        // MFMAs ahead, under the next block's mask and max.
        auto vfrag = [&](const int i) __attribute__((always_inline)) {
            const int s4 = i >> 2, db = i & 3;
            const _Float16 *vr = &Vt[vb][(32 * db + lr) * kVRow + 32 * (s4 >> 1) + 16 * (s4 & 1) + 4 * lg];
            const u32x2 v0 = *reinterpret_cast<const u32x2 *>(vr);
            const u32x2 v1 = *reinterpret_cast<const u32x2 *>(vr + 8);
            return __builtin_bit_cast(half8, u32x4{v0.x, v0.y, v1.x, v1.y});
        };
        half8 vf[kAhead + 1];
#pragma unroll
        for (int i = 0; i < kAhead; ++i) vf[i] = vfrag(i);
        float bm[2] = {-INFINITY, -INFINITY};  // two independent chains
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            o[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[i % (kAhead + 1)], pf[i >> 2], o[i & 3], 0, 0, 0);
            if (i + kAhead < 16) vf[(i + kAhead) % (kAhead + 1)] = vfrag(i + kAhead);
            // scores 2i, 2i + 1 of the next block: half i / 8, slots 2 (i % 8), + 1
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int kb2 = i >> 3, r = 2 * (i & 7) + e;
                if (mask_next) {
                    const int key = (kb + 1) * kBKV + 32 * kb2 + (r & 3) + 8 * (r >> 2) + 4 * lg;
                    if (key >= limit) sn[kb2][r] = -INFINITY;
                }
                bm[e] = fmaxf(bm[e], sn[kb2][r]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        float bmax_n;
        {
            const float bmm = fmaxf(bm[0], bm[1]);
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(bmm), __float_as_uint(bmm), false, false);
            bmax_n = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        }
        DOE_PF_STORE_K(vb);  // K(kb + 2): K(kb) was read before the previous barrier
        DOE_PF_STORE_V(kn);  // V(kb + 1): V(kb - 1) likewise
        __syncthreads();
        bmax_c = bmax_n;
    };
    float16v sn[2];
    int kb = 0;
    for (; kb + 2 < nkb_full; kb += 2) {  // two iterations whose next blocks need no mask
        iter(kb, false, sc, sn);
        iter(kb + 1, false, sn, sc);
    }
    for (; kb < nkb; ++kb) {  // the rest (a mask on blocks every query sees is a no-op)
        iter(kb, true, sc, sn);
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2) sc[kb2] = sn[kb2];
    }
    }
#undef DOE_PF_LOAD_K
#undef DOE_PF_LOAD_V
#undef DOE_PF_STORE_K
#undef DOE_PF_STORE_V

    if (qi >= a.q_len) return;
    const auto lsw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_i), __float_as_uint(l_i), false, false);
    const float l_tot = __uint_as_float(lsw[0]) + __uint_as_float(lsw[1]);
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

// Library-owned workspace (grow-only) for the f16 V^T copy.
std::mutex g_ws_mu;
void *g_ws = nullptr;
size_t g_ws_bytes = 0;

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
    DOE_REQUIRE(num_heads <= 4096 && q_len <= (1 << 24) && kv_stride <= (1 << 24) && kv_len <= (1 << 22) &&
                    num_kv_heads * kv_stride * kD <= ((int64_t)1 << 40),
                DOE_E_UNSUPPORTED, "prefill attention shape too large");
    if (q_len == 0) return DOE_OK;
    DOE_REQUIRE(q && out && (kv_len == 0 || (k && v)), DOE_E_INVALID, "null pointer");
    DOE_REQUIRE((((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15) == 0, DOE_E_INVALID,
                "q, k, v and out must be 16-byte aligned");
    PrefillArgs a;
    a.q = q;
    a.k = k;
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
        return doe::fill_bytes_async(out, 0, bytes, st);
    }
    const int64_t blocks = (int64_t)a.nqb * a.hq;
    DOE_REQUIRE(blocks <= 0x7fffffff, DOE_E_UNSUPPORTED, "too many blocks");
    const int64_t nkb_all = (kv_len + kBKV - 1) / kBKV;
    a.kv_pad = (int)(nkb_all * kBKV);
    const size_t need = (size_t)num_kv_heads * kD * (size_t)a.kv_pad * sizeof(_Float16);
    _Float16 *vt;
    {
        std::lock_guard<std::mutex> lk(g_ws_mu);
        if (g_ws_bytes < need) {
            doe::retire_workspace(g_ws);  // queued kernels and captured graphs may still use it
            g_ws = nullptr;
            g_ws_bytes = 0;
            DOE_HIP_CHECK(hipMalloc(&g_ws, need));
            g_ws_bytes = need;
        }
        vt = (_Float16 *)g_ws;
    }
    a.vt = vt;
    hipLaunchKernelGGL(v_to_f16t_kernel, dim3((unsigned)nkb_all, (unsigned)num_kv_heads), dim3(256), 0, st, v, vt,
                       a.kv_len, a.kv_stride, a.kv_pad);
    DOE_LAUNCH_CHECK("v_to_f16t_kernel");
    hipLaunchKernelGGL(attn_prefill_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a);
    DOE_LAUNCH_CHECK("attn_prefill_kernel");
    return DOE_OK;
}

}  // extern "C"
