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
//     scaled per batch row by a power of two so its max over the wave's K
//     range sits near 2^14, split into two f16), in the k order of B below;
//   * B = the nibbles of one u32 per lane as f16 subnormals with ANDs only:
//     w & 0x000F000F holds nibbles 0 and 4 as q * 2^-24, w & 0x00F000F0
//     nibbles 1 and 5 as q * 2^-20 (the image holds x / 16 there), and the
//     same of w >> 8 nibbles 2, 6 and 3, 7: every product is exact and
//     D = 2^-24 * sum(q x) of the group.
// D lands with lane (row, column group) holding four batch columns of one
// row: one f16 scale (v_fma_mix) serves all four.  The -8 of (q - 8) is one
// more MFMA per 16-row tile over the wave's eight groups: A = the group sums
// of each image column (from an MFMA of the image against ones, split into
// f16 hi and lo parts), B = the rows' f16 scales, so D_c = sum_g s * sum(x)
// and y = 2^-24 (sum_g s D_g - 8 D_c).  The power-of-two unscale per (wave,
// batch row) and the hi + lo sum (one cross-half lane swap) come at the end.
//
// Each wave builds the image of its own K range from x in its prologue (lane
// (column c, quarter kg) loads the eight x of its batch row c % 8 and group
// quarter, the max over the range meets in two lane swaps): the x loads go
// out first, then the weight loads, and the image is built while those are in
// flight.  A workgroup of the one-shot kernel owns 64 rows (four 16-row tiles
// per wave, so an image fragment feeds four MFMAs) and 32 groups of K, eight
// per wave with every load of a wave issued up front; the four waves' sums
// meet in LDS.  When K spans more than one workgroup's 32 groups, the grid
// splits K and each range writes its partial sums to a workspace: in the
// one-shot kernel the last range of a row block to finish adds the ranges in
// order (a 64-bit count per row block that only grows: the range that brings
// it to a multiple of the range count adds), in the streaming form a second
// kernel does; either way y is the same bit for bit on every run.
#include "common.h"

#include <math.h>
#include <map>
#include <mutex>

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxBatch = 8;
constexpr int kGpw = 8;  // groups per wave: one 16-byte scale load per row covers them

// B operand of one word: halves (n0, n4, 16 n1, 16 n5, n2, n6, 16 n3, 16 n7) * 2^-24.
__device__ __forceinline__ half8 unpack_int4(uint32_t w) {
    const uint32_t w8 = w >> 8;
    return __builtin_bit_cast(half8, u32x4{w & 0x000f000fu, w & 0x00f000f0u, w8 & 0x000f000fu, w8 & 0x00f000f0u});
}

// f16 hi / lo split of two floats, packed: hi = RTZ(t), lo = RTZ(t - hi);
// |t - hi| is below one f16 ulp of t, so hi + lo carries 21+ bits of t.
__device__ __forceinline__ void split_pair(const float t0, const float t1, uint32_t &hi, uint32_t &lo) {
    const auto h = __builtin_amdgcn_cvt_pkrtz(t0, t1);
    hi = __builtin_bit_cast(uint32_t, h);
    lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(t0 - (float)h[0], t1 - (float)h[1]));
}

struct Int4Args {
    const uint32_t *q;
    const uint16_t *scales;
    const float *x;  // [M][K]
    float *out;      // one K range: y [M][N]; else the ranges' partial sums
    float *y;        // [M][N]
    unsigned long long *cnt;  // one-shot kernel, K split: ranges done per row block, a multiple of the
                              // range count between calls
    int M, N, K, G;
    int xcd_map;  // 1: workgroup ids dealt so that a row block's K ranges share an XCD
};

// Workgroup id -> work item such that consecutive items run on one XCD
// (workgroups are dealt to the eight XCDs by id % 8): XCD x takes items
// [x * base + min(x, rem), + base + (x < rem)).  The K ranges of a row block
// are consecutive items, so the scale line two neighbouring ranges share
// (a range's 32 groups are 64 bytes of a 128-byte line) is fetched into one
// L2 instead of two.
__device__ __forceinline__ int xcd_item(int id, int total, int on) {
    if (!on) return id;
    const int base = total >> 3, rem = total & 7, x = id & 7;
    return x * base + min(x, rem) + (id >> 3);
}

// s_waitcnt vmcnt(0) (every load and store of the wave complete), as the
// compiler's own wait so that it tracks it; the empty asm keeps memory
// operations on their side of it.
__device__ __forceinline__ void wait_memory() {
    __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8) | (0 << 14));
    asm volatile("" ::: "memory");
}

// The x image of the wave's kGpw groups from group gb: lane (c = lane & 15,
// kg = lane >> 4) holds the A fragment of column c -- batch row c % 8, x_hi
// for c < 8 and x_lo for c >= 8 -- over elements 8 kg .. 8 kg + 7 of each
// group, in B's slot order n0 n4 n1 n5 n2 n6 n3 n7 (slots 2, 3, 6, 7 meet
// nibbles coded at bits 4..7 (x 16): they hold x / 16).  Rows past M and
// inactive waves hold zeros.  x_load issues the lane's loads (before the
// weights', so that the image is built while those are in flight); x_image
// builds the fragments and returns the lane's batch-row exponent: x was
// scaled by 2^sig.
__device__ __forceinline__ void x_load(const Int4Args &a, const int gb, const int lane, float v[kGpw][8]) {
    const int c = lane & 15, kg = lane >> 4, b = c & 7;
    const float *xr = a.x + (size_t)(b < a.M ? b : 0) * a.K + 32 * gb + 8 * kg;
#pragma unroll
    for (int u = 0; u < kGpw; ++u) {
        const float4 p0 = reinterpret_cast<const float4 *>(xr + 32 * u)[0];
        const float4 p1 = reinterpret_cast<const float4 *>(xr + 32 * u)[1];
        v[u][0] = p0.x; v[u][1] = p0.y; v[u][2] = p0.z; v[u][3] = p0.w;
        v[u][4] = p1.x; v[u][5] = p1.y; v[u][6] = p1.z; v[u][7] = p1.w;
    }
}

__device__ __forceinline__ int x_image(const Int4Args &a, const bool active, const int lane,
                                       const float v[kGpw][8], half8 xa[kGpw], half8 &ac) {
    const int c = lane & 15, kg = lane >> 4;
    const bool live = active && (c & 7) < a.M;
    float amax = 0.0f;
#pragma unroll
    for (int u = 0; u < kGpw; ++u)
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[u][j]));
    // the four quarters of the range hold batch row c % 8 in lanes c, c + 16, ...
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    int sig = 0;
    if (live && amax > 0.0f && amax <= 3.0e38f) {
        sig = 14 - __builtin_amdgcn_frexp_expf(amax);
        sig = sig < -120 ? -120 : (sig > 120 ? 120 : sig);
    }
    // columns of rows past M are zero (or NaN from x * 0 where row 0 holds an
    // infinity): every later step keeps columns apart, and they are never stored
    const float sc = live ? __builtin_amdgcn_ldexpf(1.0f, sig) : 0.0f, sc16 = sc * 0.0625f;
    const bool lo = c >= 8;
#pragma unroll
    for (int u = 0; u < kGpw; ++u) {
        uint32_t d[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            // slots 2p, 2p + 1 hold nibbles p and p + 4; pairs 1 and 3 take x / 16
            uint32_t h, l;
            const float s_ = (p & 1) ? sc16 : sc;
            split_pair(v[u][p] * s_, v[u][p + 4] * s_, h, l);
            d[p] = lo ? l : h;
        }
        xa[u] = __builtin_bit_cast(half8, u32x4{d[0], d[1], d[2], d[3]});
    }
    // A of the correction MFMA: lane (c, kg) holds, for groups u = 0..7, the
    // image column c's group sum times 2^-8 (f16 hi parts in quarter 0, lo
    // parts in quarter 1, zeros in quarters 2 and 3).  The sums come from
    // D[m][c] = sum_k ones[m][k] img[c][k] (ones = 16 on the x / 16 slots),
    // which lands column c in lanes c, c + 16, ...
    const half8 ones = {1, 1, 16, 16, 1, 1, 16, 16};
    float sx[kGpw];
#pragma unroll
    for (int u = 0; u < kGpw; ++u) {
        const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
        sx[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, xa[u], zero, 0, 0, 0)[0] * 0.00390625f;
    }
    uint32_t hc[4], lc[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) split_pair(sx[2 * p], sx[2 * p + 1], hc[p], lc[p]);
    const u32x4 zw = {0u, 0u, 0u, 0u};
    ac = __builtin_bit_cast(half8, kg == 0 ? u32x4{hc[0], hc[1], hc[2], hc[3]}
                                          : (kg == 1 ? u32x4{lc[0], lc[1], lc[2], lc[3]} : zw));
    return sig;
}

// Exponents of the four batch columns 4 lg + i (i < 4) a lane's D holds:
// batch 4 (lg & 1) + i, whose exponent lane c = batch of the image holds.
__device__ __forceinline__ void column_exponents(const int sig, const int lg, int e[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = 24 - __shfl(sig, 4 * (lg & 1) + i, 64);
}

// 64 rows x (4 kGpw) groups per workgroup: workgroup i takes row block
// i / ranges and K range sp = i % ranges (the ranges of one row block run
// side by side, so the row's bytes are read together), wave w the groups
// [sp 4 kGpw + w kGpw, + kGpw).  A row's kGpw groups are kGpw * 16
// contiguous bytes: the wave reads them with whole-line 16-byte loads (kGpw
// lanes per row) and regroups them through its own LDS slice into the MFMA
// lane order (lane (r, j) takes word j of each group of row r).  More than
// one range: the range's sums go to out[sp][M][N].
__global__ __launch_bounds__(256) void int4_gemv_kernel(Int4Args a, int ranges) {
    __shared__ float red[3][4][4][64];
    __shared__ __attribute__((aligned(16))) uint32_t wl[4][64 * 4 * kGpw];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int item = xcd_item(blockIdx.x, gridDim.x, a.xcd_map);
    const int rb = item / ranges, sp = item - rb * ranges;
    const int r0 = rb * 64;
    const int g0 = (sp * 4 + wave) * kGpw;
    const bool active = g0 < a.G;  // a.G is a multiple of kGpw
    const int gb = active ? g0 : 0;

    // x (L2-resident after the first workgroups), then the scales and weight
    // bytes (HBM); the image is built while the weights are in flight
    float xv[kGpw][8];
    x_load(a, gb, lane, xv);
    u32x4 sv[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
        sv[t] = *reinterpret_cast<const u32x4 *>(a.scales + (size_t)min(r0 + 16 * t + lr, a.N - 1) * a.G + gb);
    constexpr int RPI = 64 / kGpw;  // rows per load instruction
    u32x4 wg[kGpw];
#pragma unroll
    for (int j = 0; j < kGpw; ++j) {
        const int row = j * RPI + lane / kGpw;
        wg[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(
            a.q + (size_t)min(r0 + row, a.N - 1) * (a.K / 8) + 4 * (gb + lane % kGpw)));
    }
    half8 xa[kGpw], ac;
    const int sig = x_image(a, active, lane, xv, xa, ac);
    // regroup: row r's 32 dwords hold (word e, group u) at (8 e + u) ^ 4 sw(r),
    // sw(r) = 0 2 4 6 1 3 5 7 over r % 8: the stores (32 lanes: 4 rows x 8
    // groups) and the 16-byte reads (8 lanes: 8 rows) each fall on distinct
    // banks (unswizzled, 8 rows' words met on one bank)
    static_assert(kGpw == 8, "the swizzle assumes 32 dwords per row");
    uint32_t *my = wl[wave];
    auto swz = [](int r) __attribute__((always_inline)) { return 4 * (((r << 1) & 7) | ((r >> 2) & 1)); };
#pragma unroll
    for (int j = 0; j < kGpw; ++j) {
        const int row = j * RPI + lane / kGpw, u = lane % kGpw;
#pragma unroll
        for (int e = 0; e < 4; ++e) my[row * 32 + ((e * kGpw + u) ^ swz(row))] = wg[j][e];
    }
    // (each wave reads back only its own slice: no workgroup barrier needed)
    uint32_t w[4][kGpw];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int row = 16 * t + lr;
        const uint32_t *rowp = my + row * 32;
#pragma unroll
        for (int h = 0; h < kGpw / 4; ++h) {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(rowp + ((lg * kGpw + 4 * h) ^ swz(row)));
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
        for (int u = 0; u < kGpw; ++u) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
                const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[u], unpack_int4(w[t][u]), zero, 0, 0, 0);
                const uint32_t pair = sv[t][u >> 1];
                const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)((u & 1) ? (pair >> 16) : pair));
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(s, d[i], acc[t][i]);
            }
        }
        // the -8: sum_g s * sum(x) of the tile's rows, times -8 * 2^-24 * 2^8
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
            const float4v dc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ac, __builtin_bit_cast(half8, sv[t]), zero, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(-0.0001220703125f, dc[i], acc[t][i]);
        }
    }
    // every wave unscales its own range (exact), then the four meet in wave 0
    int e[4];
    column_exponents(sig, lg, e);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] = __builtin_amdgcn_ldexpf(acc[t][i], e[i]);
    if (wave > 0) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave - 1][t][i][lane] = acc[t][i];
    }
    __syncthreads();
    if (wave > 0) return;
    // x_hi columns sit in lanes 0..31, x_lo in 32..63: one swap adds them
    float yv[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = ((acc[t][i] + red[0][t][i][lane]) + red[1][t][i][lane]) + red[2][t][i][lane];
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            yv[t][i] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
    if (ranges == 1) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int b = 4 * lg + i, row = r0 + 16 * t + lr;
                if (lg < 2 && b < a.M && row < a.N) a.y[(size_t)b * a.N + row] = yv[t][i];
            }
        return;
    }
    // K split: the range's 512 sums ([batch][64 rows]) go to its workspace
    // slot with agent-scope stores (written through to memory); once they are
    // complete the row block's count goes up, and the workgroup that brings it
    // to a multiple of the range count adds the ranges' slots in range order
    // (agent-scope loads) into y.  No workgroup waits for another, and no
    // count is ever reset: every call adds exactly `ranges` to each of its row
    // blocks' counts (one region of counts per range count), so calls that
    // overlapped on the shared workspace (and raced on its slots) leave the
    // counts consistent for every later call.
    // Ordering: the slot stores are acknowledged (vmcnt(0)) before the count
    // is incremented, and the adding workgroup's loads are issued only after
    // its increment has returned the final count; agent-scope stores write
    // through and agent-scope loads miss the per-XCD caches, so those loads
    // read what the stores wrote.  (A release / acquire pair would say the
    // same to the compiler, but on gfx950 its agent-scope release writes back
    // the whole L2 of the XCD, measured at ~75 ns per workgroup, serialised.)
    float *slot = a.out + ((size_t)rb * ranges + sp) * 512;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (lg < 2) __hip_atomic_store(slot + (4 * lg + i) * 64 + 16 * t + lr, yv[t][i], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    wait_memory();
    unsigned long long done = 0;
    if (lane == 0) done = __hip_atomic_fetch_add(a.cnt + rb, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    done = ((unsigned long long)__builtin_amdgcn_readfirstlane((unsigned)(done >> 32)) << 32) |
           (unsigned)__builtin_amdgcn_readfirstlane((unsigned)done);
    if ((done + 1) % (unsigned)ranges != 0) return;
    asm volatile("" ::: "memory");
    // lane l, step j: batch j, row r0 + l; eight ranges' loads in flight at a time
    const float *base = a.out + (size_t)rb * ranges * 512 + lane;
    float sum[8] = {};
    for (int r0r = 0; r0r < ranges; r0r += 8) {
        float v[8][8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                v[q][j] = r0r + q < ranges
                              ? __hip_atomic_load(base + (size_t)(r0r + q) * 512 + 64 * j, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT)
                              : 0.0f;
#pragma unroll
        for (int q = 0; q < 8; ++q)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (r0r + q < ranges) sum[j] = (r0r + q == 0) ? v[q][j] : sum[j] + v[q][j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
        if (j < a.M && r0 + lane < a.N) a.y[(size_t)j * a.N + r0 + lane] = sum[j];
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

// Streaming form: a workgroup owns one K range of 4 kGpw groups (wave w the
// kGpw groups from 4 kGpw split + w kGpw) and walks the row blocks
// j, j + wps, j + 2 wps, ... of 64 rows.  The wave's x image is built once;
// each row block's weights and scales are loaded while the previous block is
// computed (two register sets), straight into the MFMA layout: lane (row, q)
// loads the 16 bytes of group 4h + q of its row and a lane-quarter transpose
// hands every lane its word of each group.  The four waves' sums meet in LDS
// (double-buffered, one barrier per block), each wave summing and storing one
// 16-row tile of the range's sums (out[split][M][N] when K is split).
template <int DEPTH>
__global__ __launch_bounds__(256, 2) void int4_gemv_stream_kernel(Int4Args a, int wps, int row_blocks) {
    __shared__ float red[DEPTH][4][4][4][64];  // [buffer][source wave][tile][column][lane]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    // With xcd_map, a few K ranges (< 8): item = j * ranges + sp, the ranges
    // walking the same row blocks neighbours on one XCD (their shared scale
    // lines fetched once); many ranges: item = sp * wps + j, each XCD holding
    // a contiguous run of ranges (so it reads its own slices of x, not all
    // of x, and neighbouring ranges still meet on one XCD but at its edges)
    const int ranges = gridDim.x / wps, item = xcd_item(blockIdx.x, gridDim.x, a.xcd_map);
    const bool range_major = !a.xcd_map || ranges >= 8;
    const int sp = range_major ? item / wps : item % ranges;
    const int j = range_major ? item - sp * wps : item / ranges;
    const int g0 = (sp * 4 + wave) * kGpw;
    const bool active = g0 < a.G;  // a.G is a multiple of kGpw
    const int gb = active ? g0 : 0;
    float *out = a.G > 4 * kGpw ? a.out + (size_t)sp * a.M * a.N : a.y;

    const size_t row_words = (size_t)a.K / 8;
    u32x4 wq[DEPTH][4][kGpw / 4], sv[DEPTH][4];
    auto load = [&](const int set, const int rb) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int row = min(rb * 64 + 16 * t + lr, a.N - 1);
            sv[set][t] = *reinterpret_cast<const u32x4 *>(a.scales + (size_t)row * a.G + gb);
#pragma unroll
            for (int h = 0; h < kGpw / 4; ++h)
                wq[set][t][h] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4 *>(a.q + row * row_words + 4 * (gb + 4 * h + lg)));
        }
    };
    int rb = j;
    if (rb >= row_blocks) return;
    float xv[kGpw][8];
    x_load(a, gb, lane, xv);
#pragma unroll
    for (int d = 0; d < DEPTH - 1; ++d)
        if (rb + d * wps < row_blocks) load(d, rb + d * wps);
    half8 xa[kGpw], ac;
    const int sig = x_image(a, active, lane, xv, xa, ac);
    int e[4];
    column_exponents(sig, lg, e);

    auto step = [&](const int cur, const int rb) __attribute__((always_inline)) {
        if (rb + (DEPTH - 1) * wps < row_blocks) load((cur + DEPTH - 1) % DEPTH, rb + (DEPTH - 1) * wps);
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
                for (int h = 0; h < kGpw / 4; ++h) {
                    uint32_t wv[4];
                    quad_transpose(wq[cur][t][h], wv);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int u = 4 * h + q;
                        const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
                        const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[u], unpack_int4(wv[q]), zero, 0, 0, 0);
                        const uint32_t pair = sv[cur][t][u >> 1];
                        const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)((u & 1) ? (pair >> 16) : pair));
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(s, d[i], acc[t][i]);
                    }
                }
                // the -8 (see the one-shot kernel)
                const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
                const float4v dc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ac, __builtin_bit_cast(half8, sv[cur][t]), zero, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(-0.0001220703125f, dc[i], acc[t][i]);
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[cur][wave][t][i][lane] = __builtin_amdgcn_ldexpf(acc[t][i], e[i]);
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
            if (lg < 2 && b < a.M && row < a.N) out[(size_t)b * a.N + row] = v;
        }
    };
    for (;;) {
        bool done = false;
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            if (!done) {
                step(d, rb);
                rb += wps;
                done = rb >= row_blocks;
            }
        }
        if (done) break;
    }
}

// y[i] = sum over the K ranges r = 0, 1, ... of part[r][i], i < M N, in range
// order; eight ranges' loads are in flight before their adds.
__global__ __launch_bounds__(256) void int4_sum_ranges_kernel(const float *__restrict__ part, float *__restrict__ y,
                                                              int64_t mn, int ranges) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= mn) return;
    float s = part[i];
    for (int r = 1; r < ranges; r += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = r + j < ranges ? part[(int64_t)(r + j) * mn + i] : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (r + j < ranges) s += v[j];
    }
    y[i] = s;
}

std::mutex g_ws_mu;
void *g_ws = nullptr;   // partial sums of the K ranges
size_t g_ws_bytes = 0;
// One-shot kernel: per range count, a region of 64-bit counts (one per row
// block), zero when allocated.
struct CountRegion {
    void *p = nullptr;
    size_t bytes = 0;
};
std::map<int, CountRegion> g_counts;
int g_num_cus = 0;
int g_int4_kernel = 0;  // 0 automatic, 1 one-shot workgroups, 2 streaming
int g_int4_depth = 3;   // streaming: row blocks in flight per wave + 1 (2 or 3)
int g_int4_plain = 0;   // 0: a row block's K ranges on one XCD, 1: workgroup ids in plain order

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
    DOE_REQUIRE(x != y, DOE_E_INVALID, "int4g32_gemv: x and y must not alias");
    if (g_num_cus == 0) {
        int dev = 0, cus = 0;
        DOE_HIP_CHECK(hipGetDevice(&dev));
        DOE_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        g_num_cus = cus > 0 ? cus : 256;
    }
    const int G = (int)(k / 32);
    const int row_blocks = (int)((n + 63) / 64);
    // eight groups per wave (every load of a wave in flight at once), K split
    // over the grid so that the rows times the ranges fill the CUs
    const int per_wg = 4 * kGpw;
    const int splits = (G + per_wg - 1) / per_wg;
    const int64_t mn = m * n;
    // the streaming form pays off once every workgroup walks several row blocks
    // (measured at batch 8: 25600 x 5120 and 5120 x 25600 faster, 9216 x 5120
    // slower than the one-shot form)
    const int64_t items = (int64_t)row_blocks * splits;
    const bool stream_ok = items >= 6 * (int64_t)g_num_cus;
    const bool one_shot = g_int4_kernel == 1 || (g_int4_kernel == 0 && !stream_ok);

    float *part = y;
    unsigned long long *cnt = nullptr;
    if (splits > 1) {
        // one-shot: [row block][range][512] slots and a count per row block;
        // streaming: [range][M][N], added by a second kernel
        const size_t need = one_shot ? (size_t)row_blocks * splits * 512 * sizeof(float)
                                     : (size_t)splits * mn * sizeof(float);
        std::lock_guard<std::mutex> lk(g_ws_mu);
        // queued kernels and captured graphs may still use the old buffers
        if (g_ws_bytes < need) {
            doe::retire_workspace(g_ws);
            g_ws = nullptr;
            g_ws_bytes = 0;
            DOE_HIP_CHECK(hipMalloc(&g_ws, need));
            g_ws_bytes = need;
        }
        part = (float *)g_ws;
        if (one_shot) {
            // the counts of this range count, zeroed once when allocated (a
            // fill kernel on this stream, so the call stays capturable)
            CountRegion &cr = g_counts[splits];
            const size_t need_cnt = (size_t)row_blocks * sizeof(unsigned long long);
            if (cr.bytes < need_cnt) {
                doe::retire_workspace(cr.p);
                cr.p = nullptr;
                cr.bytes = 0;
                DOE_HIP_CHECK(hipMalloc(&cr.p, need_cnt));
                const int frc = doe::fill_bytes_async(cr.p, 0, need_cnt, st);
                if (frc) {
                    DOE_HIP_CHECK(hipFree(cr.p));
                    cr.p = nullptr;
                    return frc;
                }
                cr.bytes = need_cnt;
            }
            cnt = (unsigned long long *)cr.p;
        }
    }
    Int4Args a;
    a.q = w_u4;
    a.scales = scales_f16;
    a.x = x;
    a.out = part;
    a.y = y;
    a.cnt = cnt;
    a.M = (int)m;
    a.N = (int)n;
    a.K = (int)k;
    a.G = G;
    a.xcd_map = !g_int4_plain;
    if (one_shot) {
        hipLaunchKernelGGL(int4_gemv_kernel, dim3((unsigned)(row_blocks * splits)), dim3(256), 0, st, a, splits);
        DOE_LAUNCH_CHECK("int4_gemv_kernel");
    } else {
        // about two workgroups per CU, each K range's row blocks dealt evenly
        const int64_t per_wg = (items + 2 * g_num_cus - 1) / (2 * g_num_cus);
        const int wps = (int)((row_blocks + per_wg - 1) / per_wg);
        if (g_int4_depth == 2)
            hipLaunchKernelGGL(int4_gemv_stream_kernel<2>, dim3((unsigned)(wps * splits)), dim3(256), 0, st, a, wps,
                               row_blocks);
        else
            hipLaunchKernelGGL(int4_gemv_stream_kernel<3>, dim3((unsigned)(wps * splits)), dim3(256), 0, st, a, wps,
                               row_blocks);
        DOE_LAUNCH_CHECK("int4_gemv_stream_kernel");
        if (splits > 1) {
            hipLaunchKernelGGL(int4_sum_ranges_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, st,
                               (const float *)part, y, mn, splits);
            DOE_LAUNCH_CHECK("int4_sum_ranges_kernel");
        }
    }
    return DOE_OK;
}

}  // extern "C"

namespace doe {

int int4_set_kernel(int v) {
    DOE_REQUIRE(v >= 0 && v <= 2, DOE_E_INVALID, "int4_gemv.kernel is 0, 1 or 2");
    g_int4_kernel = v;
    return DOE_OK;
}

int int4_set_xcd(int v) {
    DOE_REQUIRE(v == 0 || v == 1, DOE_E_INVALID, "int4_gemv.xcd is 0 (automatic) or 1 (plain workgroup order)");
    g_int4_plain = v;
    return DOE_OK;
}

int int4_set_depth(int v) {
    DOE_REQUIRE(v == 0 || v == 2 || v == 3, DOE_E_INVALID, "int4_gemv.depth is 0 (automatic), 2 or 3");
    g_int4_depth = v == 0 ? 3 : v;
    return DOE_OK;
}

}  // namespace doe
