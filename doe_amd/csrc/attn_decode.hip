// attn_decode.hip -- GQA decode attention over an f16 KV cache for gfx950.
//
// Semantics (runtime/zig/tests/tsir/real/attention_head256_f16kv/
// attention_head256_f16kv.wgsl:46-49, 72-267 and the two-pass softmax of
// runtime/zig/src/tsir/reference_interpreter.zig:1175-1265): for every query
// head h, kv head = h / (Hq / Hkv); the query sits at position kv_len - 1;
// keys [min_key, kv_len) are visible, min_key = kv_len - window when a sliding
// window is set and kv_len - 1 >= window; s = (q . k) * scale, optionally
// softcapped tanh(s / cap) * cap; o = softmax(s) V.
//
// Work decomposition: grid (splits, kv heads, batch), W waves (4; or, opt-in
// through doe_tune_set, 16 -- 8 at head_dim 256 -- as one split in one
// kernel, without the split combine).  A
// workgroup owns one kv head of one sequence and a contiguous range of
// 16-position blocks; wave w takes blocks w, w+W, ...  All G = Hq/Hkv query
// heads of the group share every K/V byte the workgroup reads.
//   * q.K^T: v_mfma_f32_16x16x32_f16 with A = the G query rows (rows >= G are
//     zero; an f32 query is split into f16 hi + lo rows accumulated by a second
//     MFMA) and B = 16 key rows (lane l reads 16 contiguous bytes of key
//     l % 16).  Lane l then holds the scores of heads 4*(l/16)+i, i < 4, for
//     position l % 16.
//   * online softmax per head inside the wave (16-lane max / sum reductions).
//   * P.V on the VALU: lane l owns dims l*D/64 .. of every head; the block's
//     probabilities are broadcast through LDS into f32 FMAs against the f16
//     V row.  Each wave prefetches its next block while computing this one.
//   * one-block form (every wave owns at most one block: short contexts,
//     the decode step): no prefetch; the query fragments held in registers;
//     with a device kv_len over a small contiguous cache, fixed block
//     ranges so the K/V loads leave before the kv_len load returns (rows
//     past the context masked, their V zeroed).
//   * the W waves combine through LDS; with more than one split, each
//     workgroup writes (m, l, o) partials to the workspace and a second,
//     small kernel combines them (a kernel boundary orders the partials
//     across XCDs far cheaper than per-workgroup release fences, which write
//     back the L2).
#include "common.h"

#include <math.h>
#include <mutex>

// The allocation-free form's split partials (doe_attn_decode_noalloc): a
// file-scope device array of kScratchBytes, one copy per GPU at its own
// address, looked up once per device by doe_init with that device current.
// Host code uses only that looked-up address (g_scratch_dev), never the
// array's name.  Every split workgroup writes its (m, l, o) partial
// unconditionally before the combine reads it, so nothing needs clearing;
// calls that overlap on one GPU share the array and race.
static constexpr size_t kScratchBytes = (size_t)16 << 20;
static constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
static float *g_scratch_dev[kMaxDevices] = {};

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct AttnArgs {
    const void *q;
    const uint16_t *k;
    const uint16_t *v;
    void *out;
    const int32_t *kv_len_dev;
    float *ws_o;       // [B*Hq][S][D] partial outputs
    float *ws_ml;      // [B*Hq][S][2] partial (max, sum)
    int q_f16, out_f16;
    int num_heads, num_kv_heads, kv_len, kv_stride, kv_layout, splits;
    int partials_only;  // write (m, l, o) partials even for one split; no combine
    float scale_log2e;  // scale * log2(e)
    float softcap;
    int sliding_window;
    int head_groups;  // workgroups per kv head, each over G of its query heads
    // Logical key p -> cache row (attention_head256_f16kv.wgsl:51-63):
    // kv_map 0: kv_start + p; 1: (kv_start + p) % ring; 2: paged, the page
    // table entry of (kv_start + p) / page_size times page_size plus the
    // offset in the page.  Rows are clamped into [0, kv_stride).
    int kv_map, kv_start, ring, page_size;
    const uint32_t *page_table;
    int page_table_len;
    // The query's absolute position: kv_start + kv_len - 1 (query_at_end) or
    // start_pos; causal keeps keys <= it, a sliding window the last `window`.
    int query_at_end, start_pos, causal;
    // > 0: split s owns the fixed blocks [s * spec_bps, (s + 1) * spec_bps),
    // at most one per wave, and each wave loads its block before the device
    // kv_len arrives (a contiguous cache whose length the host knows only as
    // kv_stride); 0: the blocks are divided by the kv_len the kernel reads.
    int spec_bps;
    // (host side) every wave owns at most one block: the launch picks the
    // kernel form without a prefetch, holding the query in registers
    int one_block;
};

constexpr int kMaxSplits = 512;
constexpr float kLazyMax = 8.0f;  // log2 headroom of the lazily raised running max

// Max / sum over each 16-lane row with DPP (quad_perm ^1, ^2, row_half_mirror,
// row_mirror): every lane of the row gets the result, no LDS round trip.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float max16(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    return fmaxf(v, dpp<0x140>(v));
}
__device__ __forceinline__ float sum16(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    return v + dpp<0x140>(v);
}

// P.V dims per lane: D / 64 for head dims that are multiples of 64, else
// four (head_dim 160: lanes 0..39 own four dims each, lanes 40..63 load a
// clamped copy of lane 39's and keep nothing).
template <int D>
constexpr int dims_per_lane() { return D % 64 == 0 ? D / 64 : 4; }
template <int D>
constexpr int v_lanes() { return D / dims_per_lane<D>(); }

// K fragment and V rows of one 16-position block, as loaded by one lane.
template <int D>
struct KVBlock {
    h8 kf[D / 32];
    _Float16 vv[16][dims_per_lane<D>()];
};

// Cache row of logical key p (see AttnArgs), clamped into the cache.
// PAGED false: the caller guarantees kv_map != 2 (no page-table load).
template <bool PAGED = true>
__device__ __forceinline__ int kv_row(const AttnArgs &a, int p) {
    const int64_t abs_key = (int64_t)a.kv_start + p;
    int64_t r = abs_key;
    if (a.kv_map == 1) {
        r = abs_key % a.ring;
    } else if (PAGED && a.kv_map == 2) {
        int64_t pg = abs_key / a.page_size;
        pg = pg < a.page_table_len ? pg : a.page_table_len - 1;
        r = (int64_t)a.page_table[pg] * a.page_size + (abs_key - (abs_key / a.page_size) * a.page_size);
    }
    return (int)(r < 0 ? 0 : (r >= a.kv_stride ? a.kv_stride - 1 : r));
}

// rowk: this lane's key row (lane l holds key p0 + l % 16); lanes 0..15 give
// the 16 rows every lane's V loads need.  A contiguous cache (vrow0 >= 0)
// passes the rows directly: position n at min(vrow0 + n, vrow_last).
template <int D>
__device__ __forceinline__ void load_block(KVBlock<D> &blk, const uint16_t *kb, const uint16_t *vb,
                                           int rowk, size_t pos_stride, int lane, int vrow0, int vrow_last) {
    constexpr int KSTEPS = D / 32, DPL = dims_per_lane<D>(), VL = v_lanes<D>();
    const int vlane = lane < VL ? lane : VL - 1;
    // dims 8 (lane / 16) + 32 s of the lane's key
    const uint16_t *krow = kb + (size_t)rowk * pos_stride + 8 * (lane >> 4);
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) blk.kf[s] = *reinterpret_cast<const h8 *>(krow + 32 * s);
    // (a select, not a branch: one straight run of loads)
#pragma unroll
    for (int n = 0; n < 16; ++n) {
        const int r = vrow0 >= 0 ? min(vrow0 + n, vrow_last) : __builtin_amdgcn_readlane(rowk, n);
        const _Float16 *vrow = reinterpret_cast<const _Float16 *>(vb + (size_t)r * pos_stride + vlane * DPL);
#pragma unroll
        for (int d = 0; d < DPL; ++d) blk.vv[n][d] = vrow[d];
    }
}

// ONE: every wave owns at most one block (no prefetch of a next block; the
// query fragments, up to head_dim 256, stay in registers).
template <int D, int G, int W, bool ONE>
__global__ __launch_bounds__(64 * W) void attn_decode_kernel(AttnArgs a) {
    constexpr int kWaves = W, kThreads = 64 * W;
    constexpr int KSTEPS = D / 32;  // MFMA k-steps over the head dimension
    constexpr int DPL = dims_per_lane<D>();  // P.V dims per lane
    constexpr int VL = v_lanes<D>();         // lanes that own P.V dims
    constexpr int G4 = (G + 3) / 4; // 4-head groups of the probability broadcast
    constexpr float kLog2e = 1.4426950408889634f;
    // Query fragments (the MFMA A operand) are staged once per workgroup in
    // LDS; the one-block form up to head_dim 256 then reads them all into
    // registers at once, before its K/V block arrives.  The wave combine and
    // the cross-split combine reuse the LDS.
    constexpr bool QREG = ONE && D <= 256;
    __shared__ union {
        h8 qfrag[2][KSTEPS][64];
        float wo[kWaves][G][D];
    } sm;
    __shared__ float4 pb[kWaves][17][G4];  // per wave: probabilities [position][head], row 16: max
    __shared__ float wm[kWaves][G], wl[kWaves][G];

    // blockIdx.y = kv head * head_groups + group: G query heads per workgroup
    const int split = blockIdx.x, kvh = (int)blockIdx.y / a.head_groups, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hq0 = (int)blockIdx.y * G;  // first query head of this group

    const size_t pos_stride = a.kv_layout == 0 ? (size_t)D : (size_t)a.num_kv_heads * D;
    const size_t kv_base = a.kv_layout == 0
                               ? ((size_t)b * a.num_kv_heads + kvh) * a.kv_stride * D
                               : (size_t)b * a.kv_stride * a.num_kv_heads * D + (size_t)kvh * D;
    const uint16_t *kb = a.k + kv_base;
    const uint16_t *vb = a.v + kv_base;

    // Query loads first (vector-memory returns are in order: staging the
    // query then never waits on the K/V stream).  Fragment s of lane l is
    // row l % 16 (query head hq0 + l % 16 when < G, else zero), dims 32 s +
    // 8 (l / 16) .. + 7.  Raw bytes first: no conversion between the loads,
    // so every query load and the first K/V block are in flight together.
    // In the one-block form two 16-byte loads per item whatever the query's
    // type (an f16 query loads its 16 bytes twice) and no branch up to the
    // K/V loads: the compiler then counts the loads still in flight exactly,
    // and converting the query waits for the query loads only.
    constexpr int QITEMS = (KSTEPS * 64 + kThreads - 1) / kThreads;
    u32x4 qraw[QITEMS][2];
#pragma unroll
    for (int it = 0; it < QITEMS; ++it) {
        const int idx = tid + it * kThreads;
        const int s = (idx >> 6) % KSTEPS, l = idx & 63, m = l & 15;
        // rows >= G (and items past the fragment count) read row 0; zeroed below
        const size_t qi = ((size_t)b * a.num_heads + hq0 + (m < G ? m : 0)) * D + 32 * s + 8 * (l >> 4);
        const char *q0 = reinterpret_cast<const char *>(a.q) + (a.q_f16 ? 2 * qi : 4 * qi);
        qraw[it][0] = *reinterpret_cast<const u32x4 *>(q0);
        if (ONE || !a.q_f16) qraw[it][1] = *reinterpret_cast<const u32x4 *>(q0 + (a.q_f16 ? 0 : 16));
    }
    KVBlock<D> cur;
    // a contiguous cache (kv_map 0) addresses V rows without lane reads
    const bool contig = a.kv_map == 0;
    int blk = 0;
    if constexpr (ONE) {
        // The wave's block from the arguments alone: with spec_bps, the fixed
        // ranges over the whole cache (rows past the visible keys are masked
        // in the scores and zeroed in V once the device kv_len is known);
        // else the host kv_len's ranges.  Rows are clamped into [0, kv_stride)
        // (the host picks this form only for kv_stride >= 1), and a wave past
        // its split's blocks loads a clamped copy it does not use.
        int hkl = a.kv_len < 0 ? 0 : a.kv_len;
        if (a.kv_map == 0 && a.kv_start == 0 && hkl > a.kv_stride) hkl = a.kv_stride;
        const int hqpos = a.query_at_end ? a.kv_start + hkl - 1 : a.start_pos;
        const int hkey_hi = !a.causal ? hkl : (hqpos < a.kv_start ? 0 : min(hkl, hqpos - a.kv_start + 1));
        const int hbps = (((hkey_hi + 15) >> 4) + a.splits - 1) / a.splits;
        const bool spec = a.spec_bps > 0;
        blk = spec ? split * a.spec_bps + wave : split * hbps + wave;
        const int hi_row = spec ? a.kv_stride - 1 : hkey_hi - 1;  // last key a lane may address
        const int rowk = kv_row<false>(a, min(blk * 16 + (lane & 15), hi_row));
        const int vlast = max(spec ? a.kv_stride - 1 : min(a.kv_start + hkey_hi - 1, a.kv_stride - 1), 0);
        const int v0 = contig ? __builtin_amdgcn_readfirstlane(min(a.kv_start + blk * 16, vlast)) : -1;
        load_block<D>(cur, kb, vb, rowk, pos_stride, lane, v0, vlast);
    }

    // a scalar load (constant address space): its wait does not include the
    // K/V loads above
    int kv_len = a.kv_len_dev ? *(const __attribute__((address_space(4))) int32_t *)a.kv_len_dev
                              : a.kv_len;
    kv_len = kv_len < 0 ? 0 : kv_len;
    if (a.kv_map == 0 && a.kv_start == 0 && kv_len > a.kv_stride) kv_len = a.kv_stride;
    // visible keys [min_key, key_hi) (attention_head256_f16kv.wgsl:115-131)
    const int qpos = a.query_at_end ? a.kv_start + kv_len - 1 : a.start_pos;
    int key_hi = kv_len, min_key = 0;
    if (a.causal) key_hi = qpos < a.kv_start ? 0 : min(kv_len, qpos - a.kv_start + 1);
    if (a.sliding_window > 0 && qpos >= a.sliding_window) {
        const int min_abs = qpos - a.sliding_window + 1;
        min_key = min_abs > a.kv_start ? min(min_abs - a.kv_start, kv_len) : 0;
    }
    const int nblk = (key_hi + 15) >> 4;
    const int bps = ONE && a.spec_bps > 0 ? a.spec_bps : (nblk + a.splits - 1) / a.splits;
    const int blk_begin = split * bps;
    const int blk_end = min(nblk, blk_begin + bps);

    const int vrow_last = min(a.kv_start + key_hi - 1, a.kv_stride - 1);
    auto vrow0 = [&](int bk) __attribute__((always_inline)) {
        return contig ? __builtin_amdgcn_readfirstlane(a.kv_start + bk * 16) : -1;
    };
    if constexpr (!ONE) {
        blk = blk_begin + wave;
        if (blk < blk_end)
            load_block<D>(cur, kb, vb, kv_row(a, min(blk * 16 + (lane & 15), key_hi - 1)), pos_stride, lane,
                          vrow0(blk), vrow_last);
    }
#pragma unroll
    for (int it = 0; it < QITEMS; ++it) {
        const int idx = tid + it * kThreads;
        if (idx < KSTEPS * 64) {
            const int s = idx >> 6, l = idx & 63, m = l & 15;
            float qv[8];
            if (a.q_f16) {
                const h8 t = __builtin_bit_cast(h8, qraw[it][0]);
#pragma unroll
                for (int j = 0; j < 8; ++j) qv[j] = (float)t[j];
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    qv[j] = __uint_as_float(qraw[it][0][j]);
                    qv[4 + j] = __uint_as_float(qraw[it][1][j]);
                }
            }
            h8 hi, lo;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float v = m < G ? qv[j] : 0.0f;
                hi[j] = (_Float16)v;
                lo[j] = (_Float16)(v - (float)hi[j]);
            }
            sm.qfrag[0][s][l] = hi;
            sm.qfrag[1][s][l] = lo;
        }
    }
    __syncthreads();
    h8 qh[QREG ? KSTEPS : 1], ql[QREG ? KSTEPS : 1];
    if constexpr (QREG) {
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
            qh[s] = sm.qfrag[0][s][lane];
            if (!a.q_f16) ql[s] = sm.qfrag[1][s][lane];
        }
    }

    float o[G][DPL];
    float mrow[G], lrow[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        mrow[h] = -INFINITY;
        lrow[h] = 0.0f;
#pragma unroll
        for (int d = 0; d < DPL; ++d) o[h][d] = 0.0f;
    }
    // running max of the heads whose scores this lane holds (4*(lane/16)+i)
    float mlane[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    const int grp = lane >> 4;
    float *pbw = reinterpret_cast<float *>(&pb[wave][0][0]);  // [17][G4*4]

    for (; blk < blk_end; blk += kWaves) {
        // Prefetch the next block of this wave while this one is computed
        // (only when there is one: a wave retires only once its loads are back).
        KVBlock<D> nxt;
        if (!ONE && blk + kWaves < blk_end)
            load_block<D>(nxt, kb, vb, kv_row(a, min((blk + kWaves) * 16 + (lane & 15), key_hi - 1)), pos_stride,
                          lane, vrow0(blk + kWaves), vrow_last);

        const int p0 = blk * 16;
        const int pk = p0 + (lane & 15);
        // the one-block form: two independent accumulation chains (even / odd
        // k-steps); the multi-block form one chain
        auto qfrag = [&](int part, int s) __attribute__((always_inline)) -> h8 {
            if constexpr (QREG) return part ? ql[s] : qh[s];
            else return sm.qfrag[part][s][lane];
        };
        f4 c0 = {0.0f, 0.0f, 0.0f, 0.0f}, c1 = c0;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
            const h8 qa = qfrag(0, s);
            if (ONE && (s & 1)) c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa, cur.kf[s], c1, 0, 0, 0);
            else c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa, cur.kf[s], c0, 0, 0, 0);
        }
        if (!a.q_f16) {
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
                const h8 qa = qfrag(1, s);
                if (ONE && (s & 1)) c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa, cur.kf[s], c1, 0, 0, 0);
                else c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa, cur.kf[s], c0, 0, 0, 0);
            }
        }
        const f4 c = c0 + c1;
        const bool valid = pk < key_hi && pk >= min_key;
        float tsum[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float s = c[i];
            if (a.softcap > 0.0f) {
                s = tanhf(s * (a.scale_log2e / kLog2e) / a.softcap) * a.softcap * kLog2e;
            } else {
                s *= a.scale_log2e;
            }
            const float sc = valid ? s : -INFINITY;  // score in log2 units
            const float m = max16(sc);
            // The running max is raised only when a block's max exceeds it by
            // more than 2^kLazyMax (probabilities then stay <= 2^kLazyMax in
            // f32), so most blocks skip the rescale of o and l below.
            const float bm = m > mlane[i] + kLazyMax ? m : mlane[i];
            mlane[i] = bm;
            const float p = valid ? __builtin_amdgcn_exp2f(sc - bm) : 0.0f;
            tsum[i] = sum16(p);
            const int h = 4 * grp + i;
            if (h < G) {
                pbw[(lane & 15) * (G4 * 4) + h] = p;
                if (!ONE && (lane & 15) == 0) pbw[16 * (G4 * 4) + h] = bm;  // new running max of head h
                if (!ONE && (lane & 15) == 1) wl[wave][h] = tsum[i];     // block sum of head h (scratch)
            }
        }
        // Head h's running max and block sum are in every lane of 16-lane
        // row h / 4 (the DPP reductions leave them there).  The one-block
        // form reads them from there (one lane read each, no LDS round trip
        // before the rescale); the multi-block form, whose next block is
        // already in flight, takes them through LDS (its lane reads measured
        // 4 % slower at 8 query heads per KV head).
        if constexpr (!ONE) __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float mnew, bsum;
            if constexpr (ONE) {
                mnew = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mlane[h & 3]), 16 * (h >> 2)));
                bsum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tsum[h & 3]), 16 * (h >> 2)));
            } else {
                mnew = pbw[16 * (G4 * 4) + h];  // the same in every lane
                bsum = wl[wave][h];
            }
            if (mnew != mrow[h]) {
                // raised from mrow (-inf before the first valid key: o and l are 0)
                const float alpha = __builtin_amdgcn_exp2f(mrow[h] - mnew);
                mrow[h] = mnew;
                lrow[h] *= alpha;
#pragma unroll
                for (int d = 0; d < DPL; ++d) o[h][d] *= alpha;
            }
            lrow[h] += bsum;
        }
        // The wave reads back the probabilities its own lanes wrote (LDS ops
        // are ordered within a wave).
        __builtin_amdgcn_wave_barrier();
        // (after the softmax, which thus overlaps the V loads' arrival)
        if (ONE && a.spec_bps > 0 && p0 + 16 > key_hi) {
            // the block past the visible keys: its rows there get probability
            // 0, and their V (never written, in a block loaded before kv_len
            // was known) is zeroed so that 0 * V stays 0.  (Other blocks
            // clamp their V rows to visible keys.  In the multi-block form
            // this branch made the compiler wait for the prefetched next
            // block before the softmax: 12 % slower at 32k keys.)
#pragma unroll
            for (int n = 0; n < 16; ++n)
                if (p0 + n >= key_hi)
#pragma unroll
                    for (int d = 0; d < DPL; ++d) cur.vv[n][d] = (_Float16)0.0f;
        }
        // P.V in batches of CH positions: the batch's probability reads all
        // go out before its FMAs (one LDS wait per batch) in the one-block
        // form up to four query heads; row by row otherwise (batches of 8
        // rows at 8 query heads per KV head measured 9 % slower, long
        // contexts)
        constexpr int CH = (ONE && G4 == 1) ? 16 : 1;
#pragma unroll
        for (int n0 = 0; n0 < 16; n0 += CH) {
            float4 pr[CH][G4];
#pragma unroll
            for (int c = 0; c < CH; ++c)
#pragma unroll
                for (int g4 = 0; g4 < G4; ++g4) pr[c][g4] = pb[wave][n0 + c][g4];
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                float pv[G4 * 4];
#pragma unroll
                for (int g4 = 0; g4 < G4; ++g4) {
                    pv[4 * g4] = pr[c][g4].x; pv[4 * g4 + 1] = pr[c][g4].y;
                    pv[4 * g4 + 2] = pr[c][g4].z; pv[4 * g4 + 3] = pr[c][g4].w;
                }
#pragma unroll
                for (int h = 0; h < G; ++h)
#pragma unroll
                    for (int d = 0; d < DPL; ++d) o[h][d] = fmaf(pv[h], (float)cur.vv[n0 + c][d], o[h][d]);
            }
        }
        __builtin_amdgcn_wave_barrier();  // pb is rewritten by the next block
        if constexpr (ONE) break;  // a single block: straight code, no loop
        cur = nxt;
    }

    // Combine the waves.
    __syncthreads();  // every wave is done with the query fragments
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            wm[wave][h] = mrow[h];
            wl[wave][h] = lrow[h];
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int d = 0; d < DPL; ++d)
            if (lane < VL) sm.wo[wave][h][lane * DPL + d] = o[h][d];
    __syncthreads();

    const size_t bh0 = (size_t)b * a.num_heads + hq0;
    for (int idx = tid; idx < G * D; idx += kThreads) {
        const int h = idx / D, d = idx % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, wm[w][h]);
        float L = 0.0f, O = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float f = __builtin_amdgcn_exp2f(wm[w][h] - M);
                L += wl[w][h] * f;
                O += sm.wo[w][h][d] * f;
            }
        }
        if (a.splits == 1 && !a.partials_only) {
            const float r = L > 0.0f ? O / L : 0.0f;
            const size_t oi = (bh0 + h) * D + d;
            if (a.out_f16) reinterpret_cast<_Float16 *>(a.out)[oi] = (_Float16)r;
            else reinterpret_cast<float *>(a.out)[oi] = r;
        } else {
            const size_t pi = (bh0 + h) * a.splits + split;
            a.ws_o[pi * D + d] = O;
            if (d == 0) {
                a.ws_ml[pi * 2] = M;
                a.ws_ml[pi * 2 + 1] = L;
            }
        }
    }
}

// Combine of the split partials: out = sum_s o_s 2^(m_s - M) / sum_s l_s
// 2^(m_s - M), M = max_s m_s.  One workgroup per (query head, 64-column
// slice of the head): thread (column quad c4, phase ph) sums splits ph,
// ph + 16, ...; its first eight splits' loads are issued before the (m, l)
// pass, and M and L are block reductions (wave shuffles, then LDS).
constexpr int kCombineCols = 64;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
    constexpr int SL = D % kCombineCols == 0 ? kCombineCols : (D < kCombineCols ? D : 32);  // columns per workgroup
    constexpr int C4 = SL / 4, PH = 256 / C4;
    constexpr int NS = D / SL;                                 // slices per head
    __shared__ float wts[kMaxSplits];
    __shared__ float4 fold[256];
    __shared__ float red[4];
    const int bh = blockIdx.x / NS, col0 = (blockIdx.x % NS) * SL, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int S = a.splits;
    const float *ml = a.ws_ml + (size_t)bh * S * 2;
    const int c4 = tid % C4, ph = tid / C4;
    const float4 *po = reinterpret_cast<const float4 *>(a.ws_o + (size_t)bh * S * D + col0) + c4;
    constexpr int DC4 = D / 4;  // float4 stride between splits

    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = po[(size_t)min(ph + u * PH, S - 1) * DC4];
    // (m, l) of splits tid and tid + 256 (S <= kMaxSplits = 512)
    float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.0f, l1 = 0.0f;
    if (tid < S) { m0 = ml[2 * tid]; l0 = ml[2 * tid + 1]; }
    if (tid + 256 < S) { m1 = ml[2 * (tid + 256)]; l1 = ml[2 * (tid + 256) + 1]; }
    float mx = wave_max(fmaxf(m0, m1));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float f0 = (m0 == -INFINITY || M == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m0 - M);
    const float f1 = (m1 == -INFINITY || M == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m1 - M);
    if (tid < S) wts[tid] = f0;
    if (tid + 256 < S) wts[tid + 256] = f1;
    const float ls = wave_sum(l0 * f0 + l1 * f1);
    __syncthreads();  // every wave has read red (M) and written wts
    if (lane == 0) red[wave] = ls;
    __syncthreads();
    const float L = (red[0] + red[1]) + (red[2] + red[3]);

    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int base = 0; base < S; base += 8 * PH) {
        if (base > 0) {
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = po[(size_t)min(base + ph + u * PH, S - 1) * DC4];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int sp = base + ph + u * PH;
            const float f = sp < S ? wts[sp] : 0.0f;
            t.x = fmaf(v[u].x, f, t.x); t.y = fmaf(v[u].y, f, t.y);
            t.z = fmaf(v[u].z, f, t.z); t.w = fmaf(v[u].w, f, t.w);
        }
    }
    fold[tid] = t;
    __syncthreads();
    if (tid < C4) {
        float4 r = fold[tid];
        for (int p2 = 1; p2 < PH; ++p2) {
            const float4 u = fold[p2 * C4 + tid];
            r.x += u.x; r.y += u.y; r.z += u.z; r.w += u.w;
        }
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        const float rv[4] = {r.x * inv, r.y * inv, r.z * inv, r.w * inv};
        const size_t oi = (size_t)bh * D + col0 + 4 * tid;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (a.out_f16) reinterpret_cast<_Float16 *>(a.out)[oi + j] = (_Float16)rv[j];
            else reinterpret_cast<float *>(a.out)[oi + j] = rv[j];
        }
    }
}

// Combine with one wave per column quad and one lane per split (S <= 64):
// lane s loads split s's (m, l) and its four columns of o, and the max and
// the sums are full-wave reductions in registers (DPP within rows, then the
// cross-row lane swaps) -- no LDS, no barrier, one memory round trip.  A
// workgroup is four waves over 16 columns of one query head.
constexpr int kWaveCombineMaxSplits = 64;

__device__ __forceinline__ float wave_max64(float v) {
    v = max16(v);
    auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
    auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
}
__device__ __forceinline__ float wave_sum64(float v) {
    v = sum16(v);
    auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
    auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
}

template <int D>
__global__ __launch_bounds__(256) void attn_combine_wave_kernel(AttnArgs a) {
    constexpr int NS = D / 16;  // 16-column slices per head
    const int bh = blockIdx.x / NS, lane = threadIdx.x & 63;
    const int col = (blockIdx.x % NS) * 16 + (threadIdx.x >> 6) * 4;
    const int S = a.splits;
    const bool on = lane < S;
    const size_t pi = (size_t)bh * S + (on ? lane : 0);
    float4 o = *reinterpret_cast<const float4 *>(a.ws_o + pi * D + col);
    float2 ml = *reinterpret_cast<const float2 *>(a.ws_ml + pi * 2);
    if (!on) {
        o = make_float4(0.f, 0.f, 0.f, 0.f);
        ml = make_float2(-INFINITY, 0.0f);
    }
    const float M = wave_max64(ml.x);
    const float f = (M == -INFINITY || ml.x == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(ml.x - M);
    const float L = wave_sum64(ml.y * f);
    const float o0 = wave_sum64(o.x * f), o1 = wave_sum64(o.y * f);
    const float o2 = wave_sum64(o.z * f), o3 = wave_sum64(o.w * f);
    if (lane == 0) {
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        const size_t oi = (size_t)bh * D + col;
        if (a.out_f16) {
            _Float16 *out = reinterpret_cast<_Float16 *>(a.out) + oi;
            out[0] = (_Float16)(o0 * inv); out[1] = (_Float16)(o1 * inv);
            out[2] = (_Float16)(o2 * inv); out[3] = (_Float16)(o3 * inv);
        } else {
            *reinterpret_cast<float4 *>(reinterpret_cast<float *>(a.out) + oi) =
                make_float4(o0 * inv, o1 * inv, o2 * inv, o3 * inv);
        }
    }
}

// Library-owned workspace (grow-only) for split partials.
std::mutex g_ws_mu;
void *g_ws = nullptr;
size_t g_ws_bytes = 0;


int g_num_cus = 0;
int g_tune_splits = 0;
int g_tune_waves = 0;
int g_tune_combine = 0;  // 0 automatic, 1 the block-reduction combine kernel

// The wide (short-context) workgroup: 16 waves up to head_dim 128, 8 at 256
// (the head-256 kernel needs more than the 128 VGPRs a 16-wave workgroup
// leaves), keeping W * G * D <= 8192 floats of wave partials in LDS.
constexpr int wide_waves(int D, int G) { return D > 256 ? 0 : (D == 256 ? 8 : 16) * (G * D <= 512 ? 1 : 0); }

template <int D, int G>
int launch_g(bool wide, dim3 grid, hipStream_t st, const AttnArgs &a) {
    constexpr int WW = wide_waves(D, G);
    if (wide && WW > 0)
        hipLaunchKernelGGL((attn_decode_kernel<D, G, (WW > 0 ? WW : 4), false>), grid, dim3(64 * WW), 0, st, a);
    else if (a.one_block)
        hipLaunchKernelGGL((attn_decode_kernel<D, G, 4, true>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((attn_decode_kernel<D, G, 4, false>), grid, dim3(256), 0, st, a);
    DOE_LAUNCH_CHECK("attn_decode_kernel");
    return DOE_OK;
}

template <int D>
int launch_main(int g, bool w, dim3 grid, hipStream_t st, const AttnArgs &a) {
    switch (g) {
        case 1: return launch_g<D, 1>(w, grid, st, a);
        case 2: return launch_g<D, 2>(w, grid, st, a);
        case 4: return launch_g<D, 4>(w, grid, st, a);
        case 6: return launch_g<D, 6>(w, grid, st, a);  // Qwen 3.6: 24 query heads on 4 KV heads
        case 8: return launch_g<D, 8>(w, grid, st, a);
        default:
            return doe::set_error(DOE_E_UNSUPPORTED, "query heads per kv head must be 1, 2, 4, 6 or 8 (got %d)", g);
    }
}

template <int D>
int launch_d(int g, bool w, dim3 grid, hipStream_t st, const AttnArgs &a) {
    int rc = launch_main<D>(g, w, grid, st, a);
    if (rc || a.splits == 1 || a.partials_only) return rc;
    const unsigned total_heads = grid.z * (unsigned)a.num_heads;
    if (a.splits <= kWaveCombineMaxSplits && g_tune_combine != 1) {
        hipLaunchKernelGGL((attn_combine_wave_kernel<D>), dim3(total_heads * (unsigned)(D / 16)), dim3(256), 0, st,
                           a);
        DOE_LAUNCH_CHECK("attn_combine_wave_kernel");
        return DOE_OK;
    }
    constexpr int SL = D % kCombineCols == 0 ? kCombineCols : (D < kCombineCols ? D : 32);
    const unsigned slices = (unsigned)(D / SL);
    hipLaunchKernelGGL((attn_combine_kernel<D>), dim3(total_heads * slices), dim3(256), 0, st, a);
    DOE_LAUNCH_CHECK("attn_combine_kernel");
    return DOE_OK;
}


}  // namespace

namespace doe {
int attn_scratch_setup(int device) {
    DOE_REQUIRE(device >= 0 && device < kMaxDevices, DOE_E_UNSUPPORTED, "device %d >= %d", device, kMaxDevices);
    if (g_scratch_dev[device]) return DOE_OK;
    void *p = nullptr;
    DOE_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    DOE_REQUIRE(p != nullptr, DOE_E_HIP, "hipGetSymbolAddress returned a null scratch address");
    g_scratch_dev[device] = static_cast<float *>(p);
    return DOE_OK;
}
int attn_set_splits(int v) {
    g_tune_splits = v;
    return DOE_OK;
}
int attn_set_waves(int v) {
    g_tune_waves = v;
    return DOE_OK;
}
int attn_set_combine(int v) {
    DOE_REQUIRE(v == 0 || v == 1, DOE_E_INVALID, "attn_decode.combine is 0 (automatic) or 1 (block reduction)");
    g_tune_combine = v;
    return DOE_OK;
}
}  // namespace doe

namespace {

// The reference attention's cache addressing and key range (defaults: the
// rows kv_start + p from 0, causal, the query at the last key).
struct KvMap {
    int kv_map = 0, kv_start = 0, ring = 0, page_size = 0;
    const uint32_t *page_table = nullptr;
    int64_t page_table_len = 0;
    int query_at_end = 1, start_pos = 0, causal = 1;
};

// parts == NULL: the library workspace and (for several splits) the combine
// kernel; parts != NULL: (o, m, l) partials into the caller's buffer
// (o [B*Hq][S][D] then ml [B*Hq][S][2]), at most max_splits splits.
int attn_decode_impl(const void *q, int q_f16, const uint16_t *k_cache, const uint16_t *v_cache,
                     void *out, int out_f16, int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                     int64_t head_dim, int64_t kv_len, const int32_t *kv_len_dev, int64_t kv_stride,
                     int kv_layout, float scale, float softcap, int64_t sliding_window,
                     float *parts, int64_t parts_capacity, int64_t max_splits_req, int32_t *splits_out,
                     doe_stream_t stream, const KvMap &map = KvMap(), float *fixed_ws = nullptr,
                     size_t fixed_ws_bytes = 0) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(batch >= 0 && num_heads > 0 && num_kv_heads > 0 && head_dim > 0 && kv_stride >= 0,
                DOE_E_INVALID, "bad attention shape");
    DOE_REQUIRE(num_heads % num_kv_heads == 0, DOE_E_INVALID,
                "num_heads %lld is not a multiple of num_kv_heads %lld", (long long)num_heads,
                (long long)num_kv_heads);
    DOE_REQUIRE(kv_layout == 0 || kv_layout == 1, DOE_E_UNSUPPORTED,
                "kv_layout %d unsupported (0: [kv_head][pos][dim], 1: [pos][kv_head][dim])", kv_layout);
    DOE_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 160 || head_dim == 256 || head_dim == 512,
                DOE_E_UNSUPPORTED, "head_dim %lld unsupported (64, 128, 160, 256, 512)", (long long)head_dim);
    const bool plain = map.kv_map == 0 && map.kv_start == 0;  // logical key p is cache row p
    DOE_REQUIRE(kv_len_dev != nullptr || (kv_len >= 0 && (!plain || kv_len <= kv_stride) && kv_len < (1 << 30)),
                DOE_E_INVALID, "kv_len %lld out of range [0, kv_stride=%lld]", (long long)kv_len,
                (long long)kv_stride);
    DOE_REQUIRE(sliding_window >= 0 && softcap >= 0.0f, DOE_E_INVALID, "negative window or softcap");
    if (batch == 0) return DOE_OK;
    DOE_REQUIRE(q && k_cache && v_cache && (out || parts), DOE_E_INVALID, "null pointer");
    DOE_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)k_cache & 15) == 0 &&
                    ((uintptr_t)v_cache & 15) == 0,
                DOE_E_INVALID, "q and the k/v caches must be 16-byte aligned");
    DOE_REQUIRE(batch * num_kv_heads <= 65535 && kv_stride <= 0x7fffffff, DOE_E_UNSUPPORTED,
                "too many sequences x kv heads");
    const int g = (int)(num_heads / num_kv_heads);
    if (g_num_cus == 0) {
        int dev = 0, cus = 0;
        DOE_HIP_CHECK(hipGetDevice(&dev));
        DOE_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        g_num_cus = cus > 0 ? cus : 256;
    }
    // Four waves and about two workgroups per CU, at least four 16-position
    // blocks each; or, when tuned so, one wide workgroup per kv head.
    const int64_t len_for_split = kv_len_dev ? kv_stride : kv_len;
    const int64_t nblk = (len_for_split + 15) / 16;
    const bool wide_ok = head_dim <= 256 && (int64_t)(num_heads / num_kv_heads) * head_dim <= 512;
    // (the wide workgroup is opt-in: at the 2B-class decode shape, head_dim
    // 256 over <= 384 positions, four-wave splits plus the combine measured
    // 767 tok/s against 742 for one eight-wave split)
    bool wide = false;
    if (g_tune_waves > 4 && wide_ok) wide = true;
    int64_t splits = (2 * g_num_cus + batch * num_kv_heads - 1) / (batch * num_kv_heads);
    // long contexts: about eight workgroups per CU (more waves streaming the
    // cache) while every split keeps at least 64 blocks (measured at batch 8,
    // 8 kv heads, 32768 positions: 8 splits 267 us, 32 splits 211-226 us)
    const int64_t splits_long = (8 * g_num_cus + batch * num_kv_heads - 1) / (batch * num_kv_heads);
    if (splits_long > splits && nblk / splits_long >= 64) splits = splits_long;
    const int64_t max_splits = (nblk + 3) / 4;
    if (wide) splits = 1;
    if (g_tune_splits > 0) splits = g_tune_splits;
    if (splits > max_splits) splits = max_splits;
    if (parts && splits > max_splits_req) splits = max_splits_req;
    if (splits > kMaxSplits) splits = kMaxSplits;
    if (splits < 1) splits = 1;

    AttnArgs a{};
    a.q = q;
    a.k = k_cache;
    a.v = v_cache;
    a.out = out;
    a.kv_len_dev = kv_len_dev;
    a.q_f16 = q_f16 != 0;
    a.out_f16 = out_f16 != 0;
    a.num_heads = (int)num_heads;
    a.num_kv_heads = (int)num_kv_heads;
    a.kv_len = (int)kv_len;
    a.kv_stride = (int)kv_stride;
    a.kv_layout = kv_layout;
    a.splits = (int)splits;
    a.scale_log2e = scale * 1.4426950408889634f;
    a.softcap = softcap;
    a.sliding_window = (int)sliding_window;
    a.kv_map = map.kv_map;
    a.kv_start = map.kv_start;
    a.ring = map.ring;
    a.page_size = map.page_size;
    a.page_table = map.page_table;
    a.page_table_len = (int)map.page_table_len;
    a.query_at_end = map.query_at_end;
    a.start_pos = map.start_pos;
    a.causal = map.causal;
    // kv_len on the device over a contiguous cache whose blocks the splits
    // cover with at most one block per wave: fixed block ranges, so every
    // wave's K/V loads leave before the kv_len load returns.
    if (kv_len_dev && plain && !wide) {
        const int64_t bps = (nblk + splits - 1) / splits;
        if (bps <= 4) a.spec_bps = (int)bps;
    }
    // at most one block per wave: the spec ranges above, or a host kv_len
    // whose blocks (nblk bounds the kernel's) divide into ranges of <= 4
    // (not over a paged cache: the one-block form reads no page table)
    a.one_block = !wide && kv_stride > 0 && map.kv_map != 2 &&
                  (a.spec_bps > 0 || (!kv_len_dev && (nblk + splits - 1) / splits <= 4));
    if (parts) {
        const int64_t o_count = batch * num_heads * splits * head_dim;
        const int64_t need = o_count + batch * num_heads * splits * 2;
        DOE_REQUIRE(parts_capacity >= need, DOE_E_INVALID,
                    "partials buffer holds %lld floats, %lld needed for %lld splits",
                    (long long)parts_capacity, (long long)need, (long long)splits);
        a.partials_only = 1;
        a.ws_o = parts;
        a.ws_ml = parts + o_count;
        if (splits_out) *splits_out = (int32_t)splits;
    } else if (splits > 1 && fixed_ws) {  // allocation-free: the caller-supplied fixed array
        const size_t o_bytes = (size_t)batch * num_heads * splits * head_dim * 4;
        const size_t ml_off = (o_bytes + 255) & ~(size_t)255;
        const size_t need = ml_off + (size_t)batch * num_heads * splits * 2 * 4;
        DOE_REQUIRE(need <= fixed_ws_bytes, DOE_E_UNSUPPORTED,
                    "split partials of %zu bytes (%lld sequences x %lld heads x %lld splits x head_dim %lld) "
                    "exceed the %zu-byte allocation-free scratch", need, (long long)batch, (long long)num_heads,
                    (long long)splits, (long long)head_dim, fixed_ws_bytes);
        a.ws_o = fixed_ws;
        a.ws_ml = (float *)((char *)fixed_ws + ml_off);
    } else if (splits > 1) {
        const size_t o_bytes = (size_t)batch * num_heads * splits * head_dim * 4;
        const size_t ml_bytes = (size_t)batch * num_heads * splits * 2 * 4;
        const size_t ml_off = (o_bytes + 255) & ~(size_t)255;
        const size_t need = ml_off + ml_bytes;
        std::lock_guard<std::mutex> lk(g_ws_mu);
        if (need > g_ws_bytes) {
            doe::retire_workspace(g_ws);  // queued kernels and captured graphs may still use it
            g_ws = nullptr;
            g_ws_bytes = 0;
            DOE_HIP_CHECK(hipMalloc(&g_ws, need));
            g_ws_bytes = need;
        }
        a.ws_o = (float *)g_ws;
        a.ws_ml = (float *)((char *)g_ws + ml_off);
    }
    // head_dim 512 holds at most two query heads per workgroup (a 16-position
    // K/V block is 64 registers per lane, double-buffered): larger groups are
    // split over g / 2 workgroups per kv head, each reading the kv head's K/V
    a.head_groups = head_dim == 512 && g > 2 ? g / 2 : 1;
    DOE_REQUIRE(num_kv_heads * a.head_groups <= 65535, DOE_E_UNSUPPORTED, "too many kv heads");
    const dim3 grid((unsigned)splits, (unsigned)(num_kv_heads * a.head_groups), (unsigned)batch);
    const hipStream_t st = (hipStream_t)stream;
    switch (head_dim) {
        case 64: return launch_d<64>(g, wide, grid, st, a);
        case 128: return launch_d<128>(g, wide, grid, st, a);
        case 160: return launch_d<160>(g, false, grid, st, a);
        case 256: return launch_d<256>(g, wide, grid, st, a);
        default:
            return launch_d<512>(g / a.head_groups, false, grid, st, a);
    }
}

}  // namespace

extern "C" {

int doe_attn_decode(const void *q, int q_f16, const uint16_t *k_cache, const uint16_t *v_cache,
                    void *out, int out_f16, int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                    int64_t head_dim, int64_t kv_len, const int32_t *kv_len_dev, int64_t kv_stride,
                    int kv_layout, float scale, float softcap, int64_t sliding_window,
                    doe_stream_t stream) {
    return attn_decode_impl(q, q_f16, k_cache, v_cache, out, out_f16, batch, num_heads, num_kv_heads,
                            head_dim, kv_len, kv_len_dev, kv_stride, kv_layout, scale, softcap,
                            sliding_window, nullptr, 0, 0, nullptr, stream);
}

int doe_attn_decode_noalloc(const void *q, int q_f16, const uint16_t *k_cache, const uint16_t *v_cache,
                            void *out, int out_f16, int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                            int64_t head_dim, int64_t kv_len, const int32_t *kv_len_dev, int64_t kv_stride,
                            int kv_layout, float scale, float softcap, int64_t sliding_window,
                            doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    int dev = -1;
    DOE_HIP_CHECK(hipGetDevice(&dev));
    DOE_REQUIRE(dev >= 0 && dev < kMaxDevices && g_scratch_dev[dev], DOE_E_NOT_INIT,
                "doe_init(%d) was not called: the allocation-free scratch of device %d is not set up", dev, dev);
    return attn_decode_impl(q, q_f16, k_cache, v_cache, out, out_f16, batch, num_heads, num_kv_heads,
                            head_dim, kv_len, kv_len_dev, kv_stride, kv_layout, scale, softcap,
                            sliding_window, nullptr, 0, 0, nullptr, stream, KvMap(), g_scratch_dev[dev],
                            kScratchBytes);
}

int doe_attention_dispatch(const doe_attention_uniforms *u, const float *q, const uint16_t *k,
                           const uint16_t *v, float *output, const uint32_t *kv_len_buffer,
                           const uint32_t *page_table, int64_t page_table_len, int64_t kv_capacity,
                           doe_stream_t stream) {
    DOE_REQUIRE(u, DOE_E_INVALID, "null uniforms");
    DOE_REQUIRE(u->kv_layout <= 2, DOE_E_INVALID, "kv_layout %u (0 contiguous, 1 ring, 2 paged)", u->kv_layout);
    DOE_REQUIRE(kv_capacity > 0 && kv_capacity < (1 << 30), DOE_E_INVALID, "kv_capacity %lld",
                (long long)kv_capacity);
    DOE_REQUIRE(u->kv_len_source == 0 || kv_len_buffer, DOE_E_INVALID, "kv_len_source 1 needs kv_len_buffer");
    DOE_REQUIRE(u->seq_len < (1u << 30) && u->kv_start < (1u << 30) && u->start_pos < (1u << 30), DOE_E_INVALID,
                "seq_len / kv_start / start_pos out of range");
    KvMap m;
    m.kv_start = (int)u->kv_start;
    if (u->kv_layout == 1 && u->sliding_window > 0) {  // ring of sliding_window rows
        DOE_REQUIRE(u->sliding_window <= kv_capacity, DOE_E_INVALID, "ring of %u rows in a %lld-row cache",
                    u->sliding_window, (long long)kv_capacity);
        m.kv_map = 1;
        m.ring = (int)u->sliding_window;
    } else if (u->kv_layout == 2) {
        DOE_REQUIRE(u->page_size > 0 && page_table && page_table_len > 0 && page_table_len < (1 << 30),
                    DOE_E_INVALID, "paged KV needs page_size > 0 and a page table");
        m.kv_map = 2;
        m.page_size = (int)u->page_size;
        m.page_table = page_table;
        m.page_table_len = page_table_len;
    }
    if (u->query_len != 1) {  // prompts: the multi-query kernel (attn_mq.hip)
        DOE_REQUIRE(u->query_len < (1u << 30), DOE_E_INVALID, "query_len %u", u->query_len);
        return doe::attention_dispatch_mq(u, q, k, v, output, kv_len_buffer, page_table, page_table_len, kv_capacity,
                                          stream);
    }
    m.query_at_end = 0;
    m.start_pos = (int)u->start_pos;
    m.causal = u->is_causal != 0;
    // K/V in the reference's [pos][kv_head][head_dim] order; f32 q and output
    return attn_decode_impl(q, 0, k, v, output, 0, 1, u->num_heads, u->num_kv_heads, u->head_dim,
                            u->kv_len_source ? 0 : (int64_t)u->seq_len,
                            u->kv_len_source ? reinterpret_cast<const int32_t *>(kv_len_buffer) : nullptr,
                            kv_capacity, 1, u->scale, u->attn_softcap, (int64_t)u->sliding_window, nullptr, 0, 0,
                            nullptr, stream, m);
}

int doe_attn_decode_partials(const void *q, int q_f16, const uint16_t *k_cache,
                             const uint16_t *v_cache, int64_t batch, int64_t num_heads,
                             int64_t num_kv_heads, int64_t head_dim, int64_t kv_len,
                             const int32_t *kv_len_dev, int64_t kv_stride, int kv_layout, float scale,
                             float softcap, int64_t sliding_window, float *partials,
                             int64_t partials_capacity, int64_t max_splits, int32_t *splits,
                             doe_stream_t stream) {
    DOE_REQUIRE(partials && max_splits >= 1 && splits, DOE_E_INVALID, "bad partials arguments");
    return attn_decode_impl(q, q_f16, k_cache, v_cache, nullptr, 0, batch, num_heads, num_kv_heads,
                            head_dim, kv_len, kv_len_dev, kv_stride, kv_layout, scale, softcap,
                            sliding_window, partials, partials_capacity, max_splits, splits, stream);
}

}  // extern "C"
