// synthetic.hip -- seeded synthetic tensors generated on the device, and the
// decode loop's on-device step bookkeeping.
//
// Benchmarks run on random-init weights of the model's shapes.  Generating
// 2+ GB of them on the host and copying them over is slow, so they are drawn
// here from a counter-based generator: element i of a tensor with seed s is a
// pure function of (s, i) (splitmix64 finaliser), so the same tensor comes out
// on every run and every device.  Normals use Box-Muller on two 24-bit
// uniforms.
#include "common.h"

#include <math.h>

namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float normal_at(uint64_t seed, uint64_t i) {
    const uint64_t r = mix64(seed * 0x632be59bd9b4e019ull + i);
    const float u1 = ((float)(r >> 40) + 1.0f) * (1.0f / 16777217.0f);  // (0, 1]
    const float u2 = (float)((r >> 16) & 0xffffffu) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
}

__global__ void fill_normal_f16_kernel(_Float16 *out, int64_t n, uint64_t seed, float mean, float sigma) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (_Float16)(mean + sigma * normal_at(seed, (uint64_t)i));
}

__global__ void fill_normal_f32_kernel(float *out, int64_t n, uint64_t seed, float mean, float sigma) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = mean + sigma * normal_at(seed, (uint64_t)i);
}

__global__ void fill_uniform_i32_kernel(int32_t *out, int64_t n, uint64_t seed, int32_t lo, int32_t hi) {
    const uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = lo + (int32_t)(mix64(seed * 0x632be59bd9b4e019ull + (uint64_t)i) % span);
}

// One thread per 16-byte word of a Q4_K_M block: word 0 holds f16 d =
// |N(0, d_sigma)| and dmin = |N(0, dmin_sigma)| plus the first 8 scale/min
// bytes, words 1..8 are uniform nibbles; the 12 scale/min bytes encode
// 6-bit values uniform in 0..63 (any byte pattern does).
__global__ void fill_q4k_kernel(uint8_t *w, int64_t nblocks, uint64_t seed, float d_sigma, float dmin_sigma) {
    const int64_t words = nblocks * 9;
    for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < words; g += (int64_t)gridDim.x * blockDim.x) {
        const int64_t blk = g / 9;
        const int word = (int)(g % 9);
        uint32_t v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint64_t r = mix64(seed * 0x632be59bd9b4e019ull + (uint64_t)g * 4 + j);
            v[j] = (uint32_t)(r >> 32);
        }
        if (word == 0) {
            const _Float16 d = (_Float16)fabsf(d_sigma * normal_at(seed ^ 0xd1b54a32d192ed03ull, (uint64_t)blk * 2));
            const _Float16 dm = (_Float16)fabsf(dmin_sigma * normal_at(seed ^ 0xd1b54a32d192ed03ull, (uint64_t)blk * 2 + 1));
            v[0] = (uint32_t)__builtin_bit_cast(uint16_t, d) | ((uint32_t)__builtin_bit_cast(uint16_t, dm) << 16);
        }
        *reinterpret_cast<uint4 *>(w + blk * DOE_Q4K_BLOCK_BYTES + word * 16) = make_uint4(v[0], v[1], v[2], v[3]);
    }
}

// Q8_0 blocks (34 bytes: f16 scale d = |N(0, d_sigma)|, 32 uniform int8
// quants), written with 2-byte stores (blocks are only 2-byte aligned).
__global__ void fill_q8_0_kernel(uint8_t *w, int64_t nblocks, uint64_t seed, float d_sigma) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nblocks;
         b += (int64_t)gridDim.x * blockDim.x) {
        uint16_t *p = reinterpret_cast<uint16_t *>(w + b * 34);
        const _Float16 d = (_Float16)fabsf(d_sigma * normal_at(seed ^ 0xd1b54a32d192ed03ull, (uint64_t)b));
        p[0] = __builtin_bit_cast(uint16_t, d);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint64_t r = mix64(seed * 0x632be59bd9b4e019ull + (uint64_t)b * 4 + j);
#pragma unroll
            for (int h = 0; h < 4; ++h) p[1 + 4 * j + h] = (uint16_t)(r >> (16 * h));
        }
    }
}

// Decode-loop bookkeeping after a step: state = [pos, kv_len, prompt_len,
// current token].  With argmax partials (one key per workgroup of the fused
// lm_head) the sampled token is their reduction (largest logit, lowest index)
// and is stored to *token first.  The next position takes the prompt token
// while inside the prompt, else the sampled token, which is also recorded in
// ids.
__global__ __launch_bounds__(256) void decode_advance_kernel(int32_t *state, int32_t *token, int32_t *ids,
                                                             int32_t max_seq,
                                                             const unsigned long long *parts, int nparts) {
    if (parts) {
        // the reference's starting point: value -FLT_MAX at index 0 (its key)
        __shared__ unsigned long long sh[4];
        unsigned long long best = ((unsigned long long)(~__float_as_uint(-3.402823466e38f)) << 32) | 0xffffffffull;
        for (int i = threadIdx.x; i < nparts; i += 256) best = parts[i] > best ? parts[i] : best;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long t = __shfl_xor(best, o, 64);
            best = t > best ? t : best;
        }
        if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            const unsigned long long a = sh[0] > sh[1] ? sh[0] : sh[1];
            const unsigned long long b = sh[2] > sh[3] ? sh[2] : sh[3];
            best = a > b ? a : b;
            token[0] = (int32_t)(0xffffffffu - (unsigned)(best & 0xffffffffull));
        }
    }
    if (threadIdx.x != 0) return;
    const int32_t next = state[0] + 1;
    if (next >= max_seq) return;
    if (next >= state[2]) ids[next] = token[0];
    state[3] = ids[next];
    state[0] = next;
    state[1] = next + 1;
}

// XOR of every 32-bit word of a buffer of n16 16-byte words: a pure read
// stream (four non-temporal 16-byte loads in flight per lane per iteration,
// one atomic XOR per workgroup at the end).  XOR commutes, so the checksum does
// not depend on the order the workgroups run in.
typedef uint32_t u32x4s __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void read_xor_kernel(const u32x4s *__restrict__ p, int64_t n16,
                                                       uint32_t *out) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        u32x4s v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < 4; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const u32x4s v = __builtin_nontemporal_load(p + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o, 64);
    // one atomic per workgroup: atomics on one address serialise
    __shared__ uint32_t wx[4];
    if ((threadIdx.x & 63) == 0) wx[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) atomicXor(out, (wx[0] ^ wx[1]) ^ (wx[2] ^ wx[3]));
}

unsigned grid_for(int64_t n) {
    int64_t b = (n + 255) / 256;
    if (b < 1) b = 1;
    return (unsigned)(b > 8192 ? 8192 : b);
}

}  // namespace

extern "C" {

int doe_fill_normal_f16(uint16_t *out, int64_t n, uint64_t seed, float mean, float sigma, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(n >= 0 && (n == 0 || out), DOE_E_INVALID, "bad fill arguments");
    if (n == 0) return DOE_OK;
    hipLaunchKernelGGL(fill_normal_f16_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                       (_Float16 *)out, n, seed, mean, sigma);
    DOE_LAUNCH_CHECK("fill_normal_f16_kernel");
    return DOE_OK;
}

int doe_fill_normal_f32(float *out, int64_t n, uint64_t seed, float mean, float sigma, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(n >= 0 && (n == 0 || out), DOE_E_INVALID, "bad fill arguments");
    if (n == 0) return DOE_OK;
    hipLaunchKernelGGL(fill_normal_f32_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, out, n,
                       seed, mean, sigma);
    DOE_LAUNCH_CHECK("fill_normal_f32_kernel");
    return DOE_OK;
}

int doe_fill_uniform_i32(int32_t *out, int64_t n, uint64_t seed, int32_t lo, int32_t hi, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(n >= 0 && (n == 0 || out) && hi > lo, DOE_E_INVALID, "bad fill arguments");
    if (n == 0) return DOE_OK;
    hipLaunchKernelGGL(fill_uniform_i32_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, out, n,
                       seed, lo, hi);
    DOE_LAUNCH_CHECK("fill_uniform_i32_kernel");
    return DOE_OK;
}

int doe_fill_random_q4k(void *weight_q4k, int64_t nblocks, uint64_t seed, float d_sigma, float dmin_sigma,
                        doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(nblocks >= 0 && (nblocks == 0 || weight_q4k), DOE_E_INVALID, "bad fill arguments");
    DOE_REQUIRE(((uintptr_t)weight_q4k & 15) == 0, DOE_E_INVALID, "weight must be 16-byte aligned");
    if (nblocks == 0) return DOE_OK;
    hipLaunchKernelGGL(fill_q4k_kernel, dim3(grid_for(nblocks * 9)), dim3(256), 0, (hipStream_t)stream,
                       (uint8_t *)weight_q4k, nblocks, seed, d_sigma, dmin_sigma);
    DOE_LAUNCH_CHECK("fill_q4k_kernel");
    return DOE_OK;
}

int doe_fill_random_q8_0(void *weight_q8_0, int64_t nblocks, uint64_t seed, float d_sigma,
                         doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(nblocks >= 0 && (nblocks == 0 || weight_q8_0), DOE_E_INVALID, "bad fill arguments");
    DOE_REQUIRE(((uintptr_t)weight_q8_0 & 1) == 0, DOE_E_INVALID, "weight must be 2-byte aligned");
    if (nblocks == 0) return DOE_OK;
    hipLaunchKernelGGL(fill_q8_0_kernel, dim3(grid_for(nblocks)), dim3(256), 0, (hipStream_t)stream,
                       (uint8_t *)weight_q8_0, nblocks, seed, d_sigma);
    DOE_LAUNCH_CHECK("fill_q8_0_kernel");
    return DOE_OK;
}

int doe_read_xor_u32(const void *buf, int64_t nbytes, uint32_t *checksum, int32_t workgroups,
                     doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(nbytes >= 0 && (nbytes & 15) == 0 && checksum && (nbytes == 0 || buf), DOE_E_INVALID,
                "read_xor needs a buffer of whole 16-byte words and a checksum pointer");
    DOE_REQUIRE(((uintptr_t)buf & 15) == 0, DOE_E_INVALID, "buffer must be 16-byte aligned");
    DOE_REQUIRE(workgroups >= 0 && workgroups <= 65536, DOE_E_INVALID, "workgroups %d", (int)workgroups);
    rc = doe::fill_bytes_async(checksum, 0, sizeof(uint32_t), (hipStream_t)stream);
    if (rc) return rc;
    if (nbytes == 0) return DOE_OK;
    const int64_t n16 = nbytes / 16;
    // automatic: up to 512 workgroups (two per CU), each lane with four
    // loads in flight per iteration (2 GiB: 7.0 TB/s at 512, 6.3 at 256,
    // 5.8-5.9 at 1024-8192 workgroups)
    int64_t grid = workgroups > 0 ? workgroups : (n16 + 1023) / 1024;
    if (grid > 512 && workgroups == 0) grid = 512;
    if (grid < 1) grid = 1;
    hipLaunchKernelGGL(read_xor_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       (const u32x4s *)buf, n16, checksum);
    DOE_LAUNCH_CHECK("read_xor_kernel");
    return DOE_OK;
}

int doe_decode_advance(int32_t *state, int32_t *token, int32_t *ids, int64_t max_seq,
                       const uint64_t *argmax_partials, int32_t num_partials, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(state && token && ids && max_seq > 0 && max_seq <= 0x7fffffff, DOE_E_INVALID,
                "bad decode_advance arguments");
    DOE_REQUIRE(!argmax_partials || num_partials > 0, DOE_E_INVALID, "no argmax partials");
    hipLaunchKernelGGL(decode_advance_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, state, token, ids,
                       (int32_t)max_seq, (const unsigned long long *)argmax_partials, (int)num_partials);
    DOE_LAUNCH_CHECK("decode_advance_kernel");
    return DOE_OK;
}

}  // extern "C"
