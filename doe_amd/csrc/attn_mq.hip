// attn_mq.hip -- multi-query (prefill) GQA attention over an f16 KV cache for
// gfx950: the query_len > 1 form of the reference attention dispatch
// (runtime/zig/tests/tsir/real/attention_head256_f16kv/
// attention_head256_f16kv.wgsl:72-267).
//
// Semantics (that file):  query i of the call sits at absolute position
// start_pos + i; it sees logical keys p in [lo_i, hi_i) where hi_i =
// min(L, abs - kv_start + 1) when causal (0 when abs < kv_start) else L, and
// lo_i = abs - window + 1 - kv_start when a sliding window is set and abs >=
// window (clamped to [0, L]), L = seq_len or kv_len_buffer[0]; logical key p
// lives in cache row kv_start + p, that modulo the window (a ring) or through
// the page table (:51-63).  Scores are q.k * scale, softcapped as
// tanh(s / cap) * cap, softmax over the visible keys; a query without keys
// writes zeros.
//
// Kernel.  One workgroup = 16 consecutive queries x HG query heads of one KV
// head (one wave per head), keys in blocks of 32 staged in LDS and shared by
// the waves: K row-major for S = Q K^T and V transposed for O = P V, both on
// v_mfma_f32_16x16x32_f16.  Q is f32: each query row is scaled by a power of
// two (max near 2^14) and split into f16 hi + lo (~22 bits), so the scores
// carry f32 quality; P is rounded to f16 once (used for both the numerator
// and the row sum).  S and O accumulators share their row mapping (lane l
// holds rows 4 (l / 16) + r), so the online-softmax rescale needs no
// exchange; row max / sum go over the 16 lanes of a DPP row.
#include "common.h"

#include <math.h>
#include <mutex>

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

struct MqArgs {
    const float *q;  // [query][num_heads][D] with q_row_stride floats per query
    const _Float16 *k, *v;
    float *out;      // [query][num_heads][D] with out_row_stride floats per query
    const uint32_t *kv_len_dev;  // non-null: L = kv_len_dev[0]
    const uint32_t *page_table;
    long row_stride, head_stride;  // halves between cache rows / kv heads
    int q_row_stride, out_row_stride;
    int num_heads, num_kv_heads, heads_per_wg, query_len, seq_len, capacity;
    int start_pos, kv_start, causal, window, kv_map, ring, page_size, page_table_len;
    float scale, softcap;
    // key split (splits > 1, grid z): split z walks its share of the query
    // block's key blocks and writes the unnormalised (o, m, l) of each row to
    // ws_o [z][query][head][D] and ws_ml [z][query][head][2]; a second kernel
    // merges them
    int splits;
    float *ws_o, *ws_ml;
};

constexpr int kKeys = 32;  // keys per block

__device__ __forceinline__ long cache_row(const MqArgs &a, int p) {
    long r = (long)a.kv_start + p;
    if (a.kv_map == 1) {
        r %= a.ring;
    } else if (a.kv_map == 2) {
        long pg = r / a.page_size;
        const long in_page = r - pg * a.page_size;
        pg = pg < a.page_table_len ? pg : a.page_table_len - 1;
        r = (long)a.page_table[pg] * a.page_size + in_page;
    }
    return r < 0 ? 0 : (r >= a.capacity ? a.capacity - 1 : r);
}

// Key range [lo, hi) of the query at absolute position abs.
__device__ __forceinline__ void key_range(const MqArgs &a, int L, long abs, int &lo, int &hi) {
    hi = L;
    if (a.causal) hi = abs < a.kv_start ? 0 : (int)min((long)L, abs - a.kv_start + 1);
    lo = 0;
    if (a.window > 0 && abs >= a.window) {
        const long mk = abs - a.window + 1;
        if (mk > a.kv_start) lo = (int)min((long)L, mk - a.kv_start);
    }
}

template <int D>
struct MqLds {
    static constexpr int QROW = D + 8, KROW = D + 8, VROW = kKeys + 8, PROW = kKeys + 8;
    static size_t bytes(int hg) {
        return ((size_t)hg * 2 * 16 * QROW + (size_t)kKeys * KROW + (size_t)D * VROW + (size_t)hg * 16 * PROW) * 2 +
               (size_t)hg * 16 * 4;
    }
};

// NTH = 64 HG threads.  A key block is staged as 16-byte pieces c = tid +
// NTH i (key c % 32, dims 8 (c / 32) ..): up to eight pieces per thread are
// fetched into registers for the next block while the current one is
// computed, the rest (head_dim 512) just before it is staged.
template <int D, int NTH>
__global__ __launch_bounds__(NTH) void attn_mq_kernel(MqArgs a) {
    using Lds = MqLds<D>;
    constexpr int PIECES = kKeys * (D / 8);
    constexpr int PPT = (PIECES + NTH - 1) / NTH;
    constexpr int PF = PPT < 8 ? PPT : 8;
    constexpr int QROW = Lds::QROW, KROW = Lds::KROW, VROW = Lds::VROW, PROW = Lds::PROW;
    constexpr int NT = D / 16;  // O tiles of 16 dims
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_raw[];
    const int HG = a.heads_per_wg;
    _Float16 *qs = reinterpret_cast<_Float16 *>(lds_raw);     // [HG][2][16][QROW]
    _Float16 *ks = qs + (size_t)HG * 2 * 16 * QROW;           // [32][KROW]
    _Float16 *vt = ks + (size_t)kKeys * KROW;                 // [D][VROW]
    _Float16 *ps = vt + (size_t)D * VROW;                     // [HG][16][PROW]
    float *qinv = reinterpret_cast<float *>(ps + (size_t)HG * 16 * PROW);  // [HG][16]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g4 = lane >> 4, c16 = lane & 15;
    const int q0 = blockIdx.x * 16;
    const int kvh = blockIdx.y / (a.num_heads / a.num_kv_heads / HG);
    const int hg = blockIdx.y % (a.num_heads / a.num_kv_heads / HG);
    const int head = kvh * (a.num_heads / a.num_kv_heads) + hg * HG + wave;
    // keys beyond what the cache addressing can hold are never visited
    // (a device length is bounded so a bad value cannot make the loop run away)
    const long lmax = a.kv_map == 0 ? (long)a.capacity - min(a.kv_start, a.capacity)
                                    : (a.kv_map == 2 ? (long)a.page_table_len * a.page_size : (1L << 24));
    const int L = (int)min(lmax, (long)(a.kv_len_dev ? a.kv_len_dev[0] : (uint32_t)a.seq_len));

    // Per-row key ranges of this lane's four rows, and the union over the 16
    // queries (the same for every head of the workgroup).
    int rlo[4], rhi[4];
    int ulo = 1 << 30, uhi = 0;
    for (int i = 0; i < 16; ++i) {
        int lo, hi;
        key_range(a, L, (long)a.start_pos + q0 + i, lo, hi);
        const bool valid = q0 + i < a.query_len;
        if (valid && hi > lo) {
            ulo = min(ulo, lo);
            uhi = max(uhi, hi);
        }
        if ((i >> 2) == g4) {
            rlo[i & 3] = valid ? lo : 0;
            rhi[i & 3] = valid ? hi : 0;
        }
    }
    const float log2e = 1.4426950408889634f;
    const _Float16 *kb = a.k + (size_t)kvh * a.head_stride;
    const _Float16 *vb = a.v + (size_t)kvh * a.head_stride;
    const _Float16 *qh = qs + (size_t)(wave * 2 + 0) * 16 * QROW;
    const _Float16 *ql = qs + (size_t)(wave * 2 + 1) * 16 * QROW;
    _Float16 *pw = ps + (size_t)wave * 16 * PROW;

    // pieces [i0, i0 + n) of the block at p0: global -> registers -> LDS
    auto fetch = [&](int p0, int i0, int n, h8 *kd, h8 *vd) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < n; ++i) {
            const int c = tid + (i0 + i) * NTH;
            const int key = c % kKeys, d0 = (c / kKeys) * 8;
            const int p = p0 + key;
            h8 kv = h8{0, 0, 0, 0, 0, 0, 0, 0}, vv = kv;
            if (c < PIECES && p < L) {
                const long row = cache_row(a, p);
                kv = *reinterpret_cast<const h8 *>(kb + row * a.row_stride + d0);
                vv = *reinterpret_cast<const h8 *>(vb + row * a.row_stride + d0);
            }
            kd[i] = kv;
            vd[i] = vv;
        }
    };
    auto put = [&](int i0, int n, const h8 *kd, const h8 *vd) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < n; ++i) {
            const int c = tid + (i0 + i) * NTH;
            if (c < PIECES) {
                const int key = c % kKeys, d0 = (c / kKeys) * 8;
                *reinterpret_cast<h8 *>(ks + (size_t)key * KROW + d0) = kd[i];
                // consecutive lanes hold consecutive keys: each V^T row's
                // writes land in consecutive halves
#pragma unroll
                for (int e = 0; e < 8; ++e) vt[(size_t)(d0 + e) * VROW + key] = vd[i][e];
            }
        }
    };
    // this split's key blocks: a contiguous share of the union's blocks
    int p0 = (ulo / kKeys) * kKeys;
    if (a.splits > 1 && p0 < uhi) {
        const int nblk = (uhi - p0 + kKeys - 1) / kKeys, per = (nblk + a.splits - 1) / a.splits;
        const int b0 = (int)blockIdx.z * per;
        uhi = min(uhi, p0 + (b0 + per) * kKeys);
        p0 += b0 * kKeys;
    }
    // the first block's loads go out before Q is read and staged
    h8 kr[PF], vr[PF];
    if (p0 < uhi) fetch(p0, 0, PF, kr, vr);
    // Q: 4 lanes per query, D / 4 dims each; per-row power-of-two scale, hi/lo.
    {
        const int i = lane >> 2, part = lane & 3;
        const int qi = q0 + i;
        const bool valid = qi < a.query_len;
        const float *src = a.q + (size_t)(valid ? qi : 0) * a.q_row_stride + (size_t)head * D + part * (D / 4);
        float amax = 0.0f;
#pragma unroll 4
        for (int d = 0; d < D / 4; d += 4) {
            const float4 f = valid ? *reinterpret_cast<const float4 *>(src + d) : make_float4(0.f, 0.f, 0.f, 0.f);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(f.x), fabsf(f.y)), fmaxf(fabsf(f.z), fabsf(f.w))));
        }
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
        int sg = 0;
        if (amax > 0.0f && amax <= 3.0e38f) {
            sg = 14 - __builtin_amdgcn_frexp_expf(amax);
            sg = sg < -100 ? -100 : (sg > 100 ? 100 : sg);
        }
        const float sc = __builtin_amdgcn_ldexpf(1.0f, sg);
        _Float16 *hrow = qs + ((size_t)(wave * 2 + 0) * 16 + i) * QROW + part * (D / 4);
        _Float16 *lrow = qs + ((size_t)(wave * 2 + 1) * 16 + i) * QROW + part * (D / 4);
#pragma unroll 2
        for (int d = 0; d < D / 4; d += 8) {
            h8 hv, lv;
#pragma unroll
            for (int e = 0; e < 8; e += 4) {
                const float4 f = valid ? *reinterpret_cast<const float4 *>(src + d + e) : make_float4(0.f, 0.f, 0.f, 0.f);
                const float t[4] = {f.x * sc, f.y * sc, f.z * sc, f.w * sc};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const _Float16 h = (_Float16)t[j];
                    hv[e + j] = h;
                    lv[e + j] = (_Float16)(t[j] - (float)h);
                }
            }
            *reinterpret_cast<h8 *>(hrow + d) = hv;
            *reinterpret_cast<h8 *>(lrow + d) = lv;
        }
        if (part == 0) qinv[wave * 16 + i] = __builtin_amdgcn_ldexpf(1.0f, -sg);
    }

    __syncthreads();
    float rowf[4];  // score scale of each row: scale / (the row's Q scale)
#pragma unroll
    for (int r = 0; r < 4; ++r) rowf[r] = a.scale * qinv[wave * 16 + 4 * g4 + r];

    f32x4 o[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m[4], l[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.0f;
    }
    for (; p0 < uhi; p0 += kKeys) {
        __syncthreads();  // every wave is done with the previous block
        put(0, PF, kr, vr);
        if constexpr (PPT > PF) {
            // the rest in chunks of eight pieces (eight loads in flight each)
#pragma unroll 1
            for (int i0 = PF; i0 < PPT; i0 += 8) {
                h8 k2[8], v2[8];
                fetch(p0, i0, 8, k2, v2);
                put(i0, 8, k2, v2);
            }
        }
        __syncthreads();
        if (p0 + kKeys < uhi) fetch(p0 + kKeys, 0, PF, kr, vr);  // in flight during this block

        // S = Q K^T: two 16-key tiles, Q hi and lo
        f32x4 s[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int c = 0; c < D / 32; ++c) {
            const h8 ah = *reinterpret_cast<const h8 *>(qh + (size_t)c16 * QROW + 32 * c + 8 * g4);
            const h8 al = *reinterpret_cast<const h8 *>(ql + (size_t)c16 * QROW + 32 * c + 8 * g4);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const h8 bk = *reinterpret_cast<const h8 *>(ks + (size_t)(16 * t + c16) * KROW + 32 * c + 8 * g4);
                s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bk, s[t], 0, 0, 0);
                s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bk, s[t], 0, 0, 0);
            }
        }
        // online softmax per row (lane holds rows 4 g4 + r, key p0 + 16 t + c16)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float x[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int p = p0 + 16 * t + c16;
                float v = s[t][r] * rowf[r];
                if (a.softcap > 0.0f) v = tanhf(v / a.softcap) * a.softcap;
                x[t] = (p >= rlo[r] && p < rhi[r]) ? v * log2e : -INFINITY;
            }
            const float bm = max16(fmaxf(x[0], x[1]));
            const float mn = fmaxf(m[r], bm);
            float corr = 1.0f;
            _Float16 ph[2] = {(_Float16)0.0f, (_Float16)0.0f};
            if (mn != -INFINITY) {
                corr = m[r] == -INFINITY ? 0.0f : exp2f(m[r] - mn);
#pragma unroll
                for (int t = 0; t < 2; ++t) ph[t] = (_Float16)(x[t] == -INFINITY ? 0.0f : exp2f(x[t] - mn));
                m[r] = mn;
            }
            l[r] = fmaf(l[r], corr, sum16((float)ph[0] + (float)ph[1]));
#pragma unroll
            for (int t = 0; t < NT; ++t) o[t][r] *= corr;
#pragma unroll
            for (int t = 0; t < 2; ++t) pw[(size_t)(4 * g4 + r) * PROW + 16 * t + c16] = ph[t];
        }
        __builtin_amdgcn_wave_barrier();
        // O += P V
        const h8 ap = *reinterpret_cast<const h8 *>(pw + (size_t)c16 * PROW + 8 * g4);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const h8 bv = *reinterpret_cast<const h8 *>(vt + (size_t)(16 * t + c16) * VROW + 8 * g4);
            o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ap, bv, o[t], 0, 0, 0);
        }
        __builtin_amdgcn_wave_barrier();  // P is rewritten by the next block
    }

#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int qi = q0 + 4 * g4 + r;
        if (qi >= a.query_len) continue;
        if (a.splits > 1) {
            const size_t pr = ((size_t)blockIdx.z * a.query_len + qi) * a.num_heads + head;
            float *dst = a.ws_o + pr * D + c16;
#pragma unroll
            for (int t = 0; t < NT; ++t) dst[16 * t] = o[t][r];
            if (c16 == 0) *reinterpret_cast<float2 *>(a.ws_ml + 2 * pr) = make_float2(m[r], l[r]);
            continue;
        }
        const float inv = l[r] > 0.0f ? 1.0f / l[r] : 0.0f;
        float *dst = a.out + (size_t)qi * a.out_row_stride + (size_t)head * D + c16;
#pragma unroll
        for (int t = 0; t < NT; ++t) dst[16 * t] = o[t][r] * inv;
    }
}

// The key splits of one (query, head) row merged: M = max m_s, L = sum l_s
// 2^(m_s - M), out = sum o_s 2^(m_s - M) / L (zero where no key was visible).
__global__ __launch_bounds__(512) void attn_mq_combine_kernel(MqArgs a, int D) {
    const int row = blockIdx.x, qi = row / a.num_heads, head = row - qi * a.num_heads, d = threadIdx.x;
    const size_t stride = (size_t)a.query_len * a.num_heads;
    float M = -INFINITY;
    for (int z = 0; z < a.splits; ++z) M = fmaxf(M, a.ws_ml[2 * (z * stride + row)]);
    float L = 0.0f, O = 0.0f;
    if (M != -INFINITY) {
        for (int z = 0; z < a.splits; ++z) {
            const float2 ml = *reinterpret_cast<const float2 *>(a.ws_ml + 2 * (z * stride + row));
            const float f = ml.x == -INFINITY ? 0.0f : exp2f(ml.x - M);
            L = fmaf(ml.y, f, L);
            O = fmaf(a.ws_o[(z * stride + row) * D + d], f, O);
        }
    }
    a.out[(size_t)qi * a.out_row_stride + (size_t)head * D + d] = L > 0.0f ? O / L : 0.0f;
}

// Key-split partials: a library-owned grow-only workspace (see the header's
// workspace rule), and the split count (0 automatic, n > 0 forced).
std::mutex g_mq_mu;
void *g_mq_ws = nullptr;
size_t g_mq_ws_bytes = 0;
int g_mq_cus = 0;
int g_mq_splits = 0;

template <int D>
int launch_mq(const MqArgs &a0, hipStream_t st) {
    MqArgs a = a0;
    const int G = a.num_heads / a.num_kv_heads;
    int hg = D <= 128 ? 8 : (D == 256 ? 4 : 2);
    while (hg > 1 && G % hg) hg >>= 1;
    if (hg > G) hg = G;
    a.heads_per_wg = hg;
    // Key split: a short prompt gives few workgroups (a 128-token prompt of
    // 4 kv heads: 32), whose last query blocks walk every key block in turn;
    // split the key blocks over the grid until about two workgroups per CU
    // (host-known key counts only: a device length keeps one split).
    const int qblocks = (a.query_len + 15) / 16, ygrid = a.num_kv_heads * (G / hg);
    if (g_mq_cus == 0) {
        int dev = 0, cus = 0;
        DOE_HIP_CHECK(hipGetDevice(&dev));
        DOE_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        g_mq_cus = cus > 0 ? cus : 256;
    }
    int splits = 1;
    if (g_mq_splits > 0) {
        splits = g_mq_splits;
    } else if (!a.kv_len_dev) {
        const long nkb = ((long)min(a.seq_len, a.capacity) + kKeys - 1) / kKeys;
        const long base = (long)qblocks * ygrid;
        if (nkb > 1 && base < g_mq_cus) {
            long sp = 2L * g_mq_cus / base;
            sp = sp < nkb ? sp : nkb;
            splits = (int)(sp < 16 ? sp : 16);
        }
    }
    a.splits = splits;
    if (splits > 1) {
        const size_t rows = (size_t)a.query_len * a.num_heads;
        const size_t o_bytes = (size_t)splits * rows * D * 4, need = o_bytes + (size_t)splits * rows * 8;
        std::lock_guard<std::mutex> lk(g_mq_mu);
        if (g_mq_ws_bytes < need) {
            doe::retire_workspace(g_mq_ws);  // queued kernels and captured graphs may still use it
            g_mq_ws = nullptr;
            g_mq_ws_bytes = 0;
            DOE_HIP_CHECK(hipMalloc(&g_mq_ws, need));
            g_mq_ws_bytes = need;
        }
        a.ws_o = (float *)g_mq_ws;
        a.ws_ml = (float *)((char *)g_mq_ws + o_bytes);
    }
    const size_t lds = MqLds<D>::bytes(hg);
    static const hipError_t attr_rc = [] {
        hipError_t e = hipSuccess;
        for (const void *f : {(const void *)attn_mq_kernel<D, 64>, (const void *)attn_mq_kernel<D, 128>,
                              (const void *)attn_mq_kernel<D, 256>, (const void *)attn_mq_kernel<D, 512>})
            if (e == hipSuccess) e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        return e;
    }();
    DOE_HIP_CHECK(attr_rc);
    DOE_REQUIRE(lds <= 160 * 1024, DOE_E_UNSUPPORTED, "attention needs %zu bytes of LDS", lds);
    const dim3 grid((unsigned)qblocks, (unsigned)ygrid, (unsigned)splits);
    switch (hg) {
        case 1: hipLaunchKernelGGL((attn_mq_kernel<D, 64>), grid, dim3(64), lds, st, a); break;
        case 2: hipLaunchKernelGGL((attn_mq_kernel<D, 128>), grid, dim3(128), lds, st, a); break;
        case 4: hipLaunchKernelGGL((attn_mq_kernel<D, 256>), grid, dim3(256), lds, st, a); break;
        default: hipLaunchKernelGGL((attn_mq_kernel<D, 512>), grid, dim3(512), lds, st, a); break;
    }
    DOE_LAUNCH_CHECK("attn_mq_kernel");
    if (splits > 1) {
        hipLaunchKernelGGL(attn_mq_combine_kernel, dim3((unsigned)(a.query_len * a.num_heads)), dim3(D), 0, st, a, D);
        DOE_LAUNCH_CHECK("attn_mq_combine_kernel");
    }
    return DOE_OK;
}

int mq_impl(MqArgs a, int64_t head_dim, hipStream_t st) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(a.num_heads > 0 && a.num_kv_heads > 0 && a.num_heads % a.num_kv_heads == 0, DOE_E_INVALID,
                "num_heads %d is not a positive multiple of num_kv_heads %d", a.num_heads, a.num_kv_heads);
    DOE_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512, DOE_E_UNSUPPORTED,
                "head_dim %lld unsupported (64, 128, 256, 512)", (long long)head_dim);
    DOE_REQUIRE(a.query_len >= 0 && a.capacity > 0, DOE_E_INVALID, "bad query_len / cache capacity");
    if (a.query_len == 0) return DOE_OK;
    DOE_REQUIRE(a.q && a.k && a.v && a.out, DOE_E_INVALID, "null pointer");
    DOE_REQUIRE(((uintptr_t)a.q & 15) == 0 && (a.q_row_stride & 3) == 0 && ((uintptr_t)a.k & 15) == 0 &&
                    ((uintptr_t)a.v & 15) == 0 && (a.row_stride & 7) == 0 && (a.head_stride & 7) == 0,
                DOE_E_INVALID, "q, k and v must be 16-byte aligned (row strides too)");
    DOE_REQUIRE(a.kv_len_dev || (a.seq_len >= 0 && (a.kv_map != 0 || a.kv_start != 0 || a.seq_len <= a.capacity)),
                DOE_E_INVALID, "seq_len %d outside the %d-row cache", a.seq_len, a.capacity);
    switch (head_dim) {
        case 64: return launch_mq<64>(a, st);
        case 128: return launch_mq<128>(a, st);
        case 256: return launch_mq<256>(a, st);
        default: return launch_mq<512>(a, st);
    }
}

}  // namespace

namespace doe {

int mq_set_splits(int value) {
    DOE_REQUIRE(value >= 0 && value <= 16, DOE_E_INVALID, "attn_mq.splits is 0..16");
    g_mq_splits = value;
    return DOE_OK;
}

// The query_len > 1 form of doe_attention_dispatch (the reference's own
// uniforms; K/V [capacity][num_kv_heads][head_dim]).
int attention_dispatch_mq(const doe_attention_uniforms *u, const float *q, const uint16_t *k, const uint16_t *v,
                          float *output, const uint32_t *kv_len_buffer, const uint32_t *page_table,
                          int64_t page_table_len, int64_t kv_capacity, doe_stream_t stream) {
    MqArgs a{};
    a.q = q;
    a.k = reinterpret_cast<const _Float16 *>(k);
    a.v = reinterpret_cast<const _Float16 *>(v);
    a.out = output;
    a.kv_len_dev = u->kv_len_source ? kv_len_buffer : nullptr;
    a.page_table = page_table;
    a.row_stride = (long)u->num_kv_heads * u->head_dim;
    a.head_stride = u->head_dim;
    a.q_row_stride = a.out_row_stride = (int)(u->num_heads * u->head_dim);
    a.num_heads = (int)u->num_heads;
    a.num_kv_heads = (int)u->num_kv_heads;
    a.query_len = (int)u->query_len;
    a.seq_len = (int)u->seq_len;
    a.capacity = (int)kv_capacity;
    a.start_pos = (int)u->start_pos;
    a.kv_start = (int)u->kv_start;
    a.causal = u->is_causal != 0;
    a.window = (int)u->sliding_window;
    if (u->kv_layout == 1 && u->sliding_window > 0) {
        a.kv_map = 1;
        a.ring = (int)u->sliding_window;
    } else if (u->kv_layout == 2) {
        a.kv_map = 2;
        a.page_size = (int)u->page_size;
        a.page_table_len = (int)page_table_len;
    }
    a.scale = u->scale;
    a.softcap = u->attn_softcap;
    return mq_impl(a, u->head_dim, (hipStream_t)stream);
}

}  // namespace doe

extern "C" int doe_attn_prefill_f16kv(const float *q, int64_t q_row_stride, const uint16_t *k_cache,
                                      const uint16_t *v_cache, float *output, int64_t out_row_stride,
                                      int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t query_len,
                                      int64_t kv_len, int64_t kv_stride, int kv_layout, int64_t start_pos,
                                      float scale, float softcap, int64_t sliding_window, doe_stream_t stream) {
    DOE_REQUIRE(kv_layout == 0 || kv_layout == 1, DOE_E_UNSUPPORTED,
                "kv_layout %d (0: [kv_head][pos][dim], 1: [pos][kv_head][dim])", kv_layout);
    DOE_REQUIRE(num_heads > 0 && num_kv_heads > 0 && head_dim > 0 && query_len >= 0 && kv_stride > 0 &&
                    kv_len >= 0 && kv_len <= kv_stride && start_pos >= 0 && sliding_window >= 0 &&
                    q_row_stride >= num_heads * head_dim && out_row_stride >= num_heads * head_dim &&
                    kv_stride < (1 << 30) && query_len < (1 << 30) && start_pos < (1 << 30),
                DOE_E_INVALID, "bad prefill attention shape");
    MqArgs a{};
    a.q = q;
    a.k = reinterpret_cast<const _Float16 *>(k_cache);
    a.v = reinterpret_cast<const _Float16 *>(v_cache);
    a.out = output;
    a.row_stride = kv_layout == 0 ? head_dim : num_kv_heads * head_dim;
    a.head_stride = kv_layout == 0 ? kv_stride * head_dim : head_dim;
    a.q_row_stride = (int)q_row_stride;
    a.out_row_stride = (int)out_row_stride;
    a.num_heads = (int)num_heads;
    a.num_kv_heads = (int)num_kv_heads;
    a.query_len = (int)query_len;
    a.seq_len = (int)kv_len;
    a.capacity = (int)kv_stride;
    a.start_pos = (int)start_pos;
    a.causal = 1;
    a.window = (int)sliding_window;
    a.scale = scale;
    a.softcap = softcap;
    return mq_impl(a, head_dim, (hipStream_t)stream);
}
