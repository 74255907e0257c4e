// ssm.hip -- the gated-DeltaNet body ops and gated activations of the
// reference's Qwen 3.6 step graph (runtime/zig/examples/execution-v1/
// qwen-3-6-27b-smoke.json: conv1d_depthwise -> l2_normalize(q, k) ->
// linear_attention per SSM layer; o_gate (sigmoid_gated) and silu_gated in
// the attention layers), for gfx950.
//
// Semantics follow the reference interpreter (runtime/zig/src/tsir/
// reference_interpreter.zig):
//   gated (:954-1052)         out = act(gate) * input; gelu with the inner
//                             argument clamped to [-15, 15], silu x / (1 +
//                             exp(z)) and sigmoid 1 / (1 + exp(z)) with z =
//                             clamp(-x, -15, 15).
//   l2_normalize (:1284-1361) per row, out = x / sqrt(sum x^2 + eps).
//   conv1d_depthwise          causal depthwise conv over [token][channel],
//     (:1363-1455)            weight [channel][kernel_size], optional bias:
//                             out[t][c] = bias[c] + sum_k in[t-(K-1-k)][c]
//                             w[c][k], the products and sums rounded in that
//                             order (bit for bit the interpreter's f32 loop).
//   linear_attention          the single-query shared-norm gated DeltaNet
//     (:1457-1596)            form: per head, alpha = 1 - exp(-A_log),
//                             for every state row d: dot = S[d] . k,
//                             S[d] = (1 - alpha) S[d] + alpha (q[d] - dot) k,
//                             out[d] = S[d] . v + sigmoid(g[d]) q[d];
//                             tokens run in order through one state.
//
// linear_attention layout: the state of a head is [value_dim][key_dim] f32
// (row d is one query / output dimension); a 16-lane row group holds one row
// in registers (key_dim / 16 values per lane) for the whole token sequence,
// the dot products are DPP sums within the group, four rows per wave, sixteen
// per workgroup; k and v of a token are loaded once per wave (every group of
// the wave reads the same key_dim floats, from L2), the next token's loads
// issued before the current token is computed.  The state is read once and
// written once per call however many tokens it covers.
#include "common.h"

#include <math.h>

namespace {

// DPP exchanges within 16-lane rows: quad_perm [1,0,3,2], [2,3,0,1],
// row_half_mirror, row_mirror; every lane of the row ends with the sum.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float sum16(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    return v + dpp<0x140>(v);
}

__device__ __forceinline__ float gated_act(float x, int kind) {
    if (kind == 0) return doe_gelu_tanh_clamped(x);
    const float z = fminf(fmaxf(-x, -15.0f), 15.0f);
    return (kind == 1 ? x : 1.0f) / (1.0f + expf(z));
}

__global__ __launch_bounds__(256) void gated_kernel(const float *__restrict__ gate, const float *__restrict__ input,
                                                    float *__restrict__ out, int64_t n, int kind) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        out[i] = gated_act(gate[i], kind) * input[i];
}

// One wave per row: lanes stride over the row, a full-wave sum of squares.
__global__ __launch_bounds__(256) void l2_normalize_kernel(const float *__restrict__ in, float *__restrict__ out,
                                                           int64_t rows, int hidden, float eps) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;  // wave-uniform
    const float *x = in + row * hidden;
    float sq = 0.0f;
    for (int d = lane; d < hidden; d += 64) sq = fmaf(x[d], x[d], sq);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o, 64);
    const float inv = 1.0f / sqrtf(sq + eps);
    for (int d = lane; d < hidden; d += 64) out[row * hidden + d] = x[d] * inv;
}

// One thread per (token, channel), channels fastest: every load coalesced.
__global__ __launch_bounds__(256) void conv1d_depthwise_kernel(const float *__restrict__ in,
                                                               const float *__restrict__ w,
                                                               const float *__restrict__ bias,
                                                               float *__restrict__ out, int64_t tokens,
                                                               int64_t channels, int kernel_size) {
    // product then sum, each rounded: no fused multiply-add (HIP's default
    // contracts a * b + c into one fma, __fmul_rn / __fadd_rn included)
#pragma clang fp contract(off)
    const int64_t total = tokens * channels;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t t = i / channels, c = i - t * channels;
        float acc = bias ? bias[c] : 0.0f;
        for (int k = 0; k < kernel_size; ++k) {
            const int64_t ti = t - (kernel_size - 1 - k);
            if (ti < 0) continue;
            const float prod = in[ti * channels + c] * w[c * kernel_size + k];
            acc = acc + prod;
        }
        out[i] = acc;
    }
}

// KPL state values per lane (key_dim <= 16 KPL); a workgroup = 16 rows of
// one head.
template <int KPL>
__global__ __launch_bounds__(256) void linear_attention_kernel(const float *__restrict__ q,
                                                               const float *__restrict__ k,
                                                               const float *__restrict__ v,
                                                               const float *__restrict__ gate, float *state,
                                                               float *__restrict__ out, int tokens, int heads,
                                                               int key_dim, int value_dim,
                                                               const float *__restrict__ a_log) {
    const int h = blockIdx.y, lane = threadIdx.x & 63, j0 = lane & 15;
    const int d = blockIdx.x * 16 + (threadIdx.x >> 4);  // this group's state row
    const bool row_ok = d < value_dim;
    const int dr = row_ok ? d : value_dim - 1;
    const float al = a_log ? a_log[h] : 0.5f;
    const float alpha = 1.0f - expf(-al), decay = 1.0f - alpha;
    float *S = state + ((size_t)h * value_dim + dr) * key_dim;
    float s[KPL], kk[KPL], vv[KPL], kn[KPL] = {}, vn[KPL] = {};
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
        const int j = j0 + 16 * i;
        s[i] = j < key_dim ? S[j] : 0.0f;
    }
    auto load_kv = [&](int t, float *kd, float *vd) __attribute__((always_inline)) {
        const float *kt = k + ((size_t)t * heads + h) * key_dim;
        const float *vt = v + ((size_t)t * heads + h) * key_dim;
#pragma unroll
        for (int i = 0; i < KPL; ++i) {
            const int j = j0 + 16 * i;
            kd[i] = j < key_dim ? kt[j] : 0.0f;
            vd[i] = j < key_dim ? vt[j] : 0.0f;
        }
    };
    if (tokens > 0) load_kv(0, kk, vv);
    for (int t = 0; t < tokens; ++t) {
        const size_t qi = ((size_t)t * heads + h) * value_dim + dr;
        const float qd = q[qi], gd = gate[qi];
        if (t + 1 < tokens) load_kv(t + 1, kn, vn);  // in flight while this token is computed
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < KPL; ++i) dot = fmaf(s[i], kk[i], dot);
        dot = sum16(dot);
        const float scaled = alpha * (qd - dot);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < KPL; ++i) {
            s[i] = fmaf(decay, s[i], scaled * kk[i]);
            acc = fmaf(s[i], vv[i], acc);
        }
        acc = sum16(acc);
        if (j0 == 0 && row_ok) out[qi] = acc + qd / (1.0f + expf(-gd));
#pragma unroll
        for (int i = 0; i < KPL; ++i) {
            kk[i] = kn[i];
            vv[i] = vn[i];
        }
    }
    if (row_ok) {
#pragma unroll
        for (int i = 0; i < KPL; ++i) {
            const int j = j0 + 16 * i;
            if (j < key_dim) S[j] = s[i];
        }
    }
}

unsigned grid_for(int64_t n) {
    int64_t b = (n + 255) / 256;
    if (b < 1) b = 1;
    return (unsigned)(b > 8192 ? 8192 : b);
}

}  // namespace

extern "C" {

int doe_gated(const float *gate, const float *input, float *output, int64_t n, int kind, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(n >= 0, DOE_E_INVALID, "negative length");
    DOE_REQUIRE(kind >= 0 && kind <= 2, DOE_E_INVALID, "kind %d (0 gelu, 1 silu, 2 sigmoid)", kind);
    if (n == 0) return DOE_OK;
    DOE_REQUIRE(gate && input && output, DOE_E_INVALID, "null pointer");
    hipLaunchKernelGGL(gated_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, gate, input, output, n,
                       kind);
    DOE_LAUNCH_CHECK("gated_kernel");
    return DOE_OK;
}

int doe_l2_normalize(const float *input, float *output, int64_t rows, int64_t hidden, float eps,
                     doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(rows >= 0 && hidden > 0 && hidden <= 0x7fffffff && eps >= 0.0f, DOE_E_INVALID,
                "bad l2_normalize shape");
    if (rows == 0) return DOE_OK;
    DOE_REQUIRE(input && output, DOE_E_INVALID, "null pointer");
    DOE_REQUIRE((rows + 3) / 4 <= 0x7fffffff, DOE_E_UNSUPPORTED, "too many rows");
    hipLaunchKernelGGL(l2_normalize_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                       input, output, rows, (int)hidden, eps);
    DOE_LAUNCH_CHECK("l2_normalize_kernel");
    return DOE_OK;
}

int doe_conv1d_depthwise(const float *input, const float *weight, const float *bias, float *output,
                         int64_t tokens, int64_t channels, int64_t kernel_size, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(tokens >= 0 && channels > 0 && kernel_size > 0 && kernel_size <= 1024, DOE_E_INVALID,
                "bad conv1d_depthwise shape");
    if (tokens == 0) return DOE_OK;
    DOE_REQUIRE(input && weight && output, DOE_E_INVALID, "null pointer");
    DOE_REQUIRE(output != input, DOE_E_INVALID, "the output must not alias the input");
    hipLaunchKernelGGL(conv1d_depthwise_kernel, dim3(grid_for(tokens * channels)), dim3(256), 0,
                       (hipStream_t)stream, input, weight, bias, output, tokens, channels, (int)kernel_size);
    DOE_LAUNCH_CHECK("conv1d_depthwise_kernel");
    return DOE_OK;
}

int doe_linear_attention(const float *q, const float *k, const float *v, const float *gate, float *state,
                         float *output, int64_t tokens, int64_t heads, int64_t key_dim, int64_t value_dim,
                         const float *a_log, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(tokens >= 0 && tokens <= 0x7fffffff && heads > 0 && heads <= 65535 && key_dim > 0 &&
                    value_dim > 0 && value_dim <= (1 << 24),
                DOE_E_INVALID, "bad linear_attention shape");
    DOE_REQUIRE(key_dim <= 256, DOE_E_UNSUPPORTED, "key_dim %lld > 256", (long long)key_dim);
    DOE_REQUIRE(q && k && v && gate && state && (output || tokens == 0), DOE_E_INVALID, "null pointer");
    const dim3 grid((unsigned)((value_dim + 15) / 16), (unsigned)heads);
    const hipStream_t st = (hipStream_t)stream;
#define DOE_LA(KPL)                                                                                        \
    hipLaunchKernelGGL(linear_attention_kernel<KPL>, grid, dim3(256), 0, st, q, k, v, gate, state, output, \
                       (int)tokens, (int)heads, (int)key_dim, (int)value_dim, a_log)
    if (key_dim <= 64) DOE_LA(4);
    else if (key_dim <= 128) DOE_LA(8);
    else DOE_LA(16);
#undef DOE_LA
    DOE_LAUNCH_CHECK("linear_attention_kernel");
    return DOE_OK;
}

}  // extern "C"
