/*
 * doe_oracle.c -- CPU oracle for the quantized-decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY: a plain-C restatement of the reference's CPU
 * evaluation of each kernel, used by tests/, the smoke check and bench.py's
 * cpu_baseline leg to check results.  It is never linked into, loaded by or
 * called from the product library.
 *
 * Reference sources restated here (paths relative to the doerun/doe root):
 *   bench/tools/doppler_rdrr_q4k.py                 Q4_K_M unpack / dequant
 *   runtime/zig/src/tsir/reference_interpreter.zig  f32 left-fold GEMV, RMSNorm,
 *                                                   gated activations, attention,
 *                                                   dtype conversions
 *   bench/tools/run_csl_webgpu_emulator.mjs         RoPE pairs, KV write, sample,
 *                                                   gather, GELU, residual
 *   bench/inference-pipeline/kernels/{rmsnorm,rope,gelu_gated,sample}.wgsl
 *                                                   index math
 *   runtime/zig/tests/tsir/real/attention_head256_f16kv/attention_head256_f16kv.wgsl
 *                                                   GQA head mapping, causal and
 *                                                   sliding-window limits, softcap
 *   runtime/zig/tests/tsir/real/lm_head_gemv/lm_head_gemv.wgsl   f16-weight GEMV
 *   runtime/zig/src/tsir/reference_interpreter.zig:954-1052, 1284-1596
 *                                                   gated activations, l2_normalize,
 *                                                   conv1d_depthwise, linear_attention
 *   bench/kernels/compilation-corpus/complex_fused_gemv_dequant.wgsl  int4 group GEMV
 *
 * Build: gcc -O2 -ffp-contract=off -fPIC -shared (see oracle/Makefile).
 */
#include "doe_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* Scalar conversions.                                                        */
/* reference_interpreter.zig:2101-2127 (readF32FromBytes: f16 upcast, bf16 is  */
/* the high half of an f32), :2162-2205 (writeF32AsElem, f32ToBf16Rne).       */
/* ------------------------------------------------------------------------- */

static float bits_to_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t f32_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

float ora_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        /* zero or subnormal: value = man * 2^-24, exact in f32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) {
        return bits_to_f32(sign | 0x7f800000u | (man << 13));
    }
    return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t ora_f32_to_f16(float f) {
    uint32_t x = f32_to_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) {
        /* inf or nan */
        return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
    }
    if (absx >= 0x477ff000u) {
        /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (absx < 0x38800000u) {
        /* result is subnormal (or zero) in f16: value / 2^-24, RNE */
        float a = bits_to_f32(absx);
        /* a * 2^24 is exact in double; rint uses the current (nearest-even) mode */
        double scaled = (double)a * 16777216.0;
        double r = rint(scaled);
        return (uint16_t)(sign | (uint32_t)r);
    }
    /* normal: keep 10 mantissa bits with RNE on the dropped 13 */
    uint32_t exp = ((absx >> 23) - 112u);
    uint32_t man = absx & 0x7fffffu;
    uint32_t half = (exp << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) {
        half += 1u; /* may carry into the exponent, which is the correct result */
    }
    return (uint16_t)(sign | half);
}

float ora_bf16_to_f32(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

uint16_t ora_f32_to_bf16(float f) {
    uint32_t bits = f32_to_bits(f);
    uint32_t exp = (bits >> 23) & 0xffu;
    uint32_t man = bits & 0x7fffffu;
    if (exp == 0xffu && man != 0) {
        return (uint16_t)((bits >> 16) | 0x40u);
    }
    uint32_t lsb = (bits >> 16) & 1u;
    uint32_t rounded = bits + 0x7fffu + lsb;
    return (uint16_t)(rounded >> 16);
}

/* ------------------------------------------------------------------------- */
/* Q4_K_M.  doppler_rdrr_q4k.py:11-15 (constants), :56-76 (scale/min bits),  */
/* :79-101 (block dequant), :128-156 (row-wise dequant with tail truncation). */
/* ------------------------------------------------------------------------- */

#define Q4K_BLOCK_BYTES 144
#define Q4K_BLOCK_ELEMS 256

void ora_q4k_unpack_scale_min(const uint8_t *b, uint8_t sc[8], uint8_t mn[8], float *d,
                              float *dmin) {
    /* doppler_rdrr_q4k.py:56-76: the first four sub-blocks take the low six
     * bits of bytes 4..7 (scales) and 8..11 (mins); the last four take a low
     * nibble from bytes 12..15 plus the top two bits of the first group. */
    *d = ora_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    *dmin = ora_f16_to_f32((uint16_t)(b[2] | (b[3] << 8)));
    for (int j = 0; j < 4; ++j) {
        sc[j] = b[4 + j] & 0x3f;
        mn[j] = b[8 + j] & 0x3f;
        sc[j + 4] = (uint8_t)((((b[4 + j] >> 6) & 0x03) << 4) | (b[12 + j] & 0x0f));
        mn[j + 4] = (uint8_t)((((b[8 + j] >> 6) & 0x03) << 4) | ((b[12 + j] >> 4) & 0x0f));
    }
}

void ora_q4k_dequant_block(const uint8_t *b, float out[256]) {
    /* doppler_rdrr_q4k.py:79-101.  The Python computes d*sc*q - dmin*m in
     * f64; every product is exact there (d, dmin are f16, sc, m < 64,
     * q < 16) and so is the difference (its span is < 53 bits), so storing
     * the result as f32 rounds the exact value once.  Compute the same
     * exact value in double and round once. */
    uint8_t sc[8], mn[8];
    float d, dmin;
    ora_q4k_unpack_scale_min(b, sc, mn, &d, &dmin);
    for (int chunk = 0; chunk < 4; ++chunk) {
        int lo_sub = 2 * chunk, hi_sub = 2 * chunk + 1;
        double s_lo = (double)d * sc[lo_sub], m_lo = (double)dmin * mn[lo_sub];
        double s_hi = (double)d * sc[hi_sub], m_hi = (double)dmin * mn[hi_sub];
        for (int i = 0; i < 32; ++i) {
            uint8_t packed = b[16 + chunk * 32 + i];
            out[chunk * 64 + i] = (float)(s_lo * (packed & 0x0f) - m_lo);
            out[chunk * 64 + 32 + i] = (float)(s_hi * ((packed >> 4) & 0x0f) - m_hi);
        }
    }
}

int ora_q4k_dequant_rowwise(const uint8_t *w, int64_t rows, int64_t cols, float *out) {
    /* doppler_rdrr_q4k.py:128-156: blocks_per_row = ceil(cols/256), row
     * stride blocks_per_row*144 bytes, each row truncated to cols values. */
    if (rows < 0 || cols < 0) return -1;
    int64_t nb = (cols + Q4K_BLOCK_ELEMS - 1) / Q4K_BLOCK_ELEMS;
    float tmp[256];
    for (int64_t r = 0; r < rows; ++r) {
        const uint8_t *row = w + (size_t)r * (size_t)nb * Q4K_BLOCK_BYTES;
        for (int64_t blk = 0; blk < nb; ++blk) {
            ora_q4k_dequant_block(row + blk * Q4K_BLOCK_BYTES, tmp);
            int64_t base = blk * Q4K_BLOCK_ELEMS;
            int64_t n = cols - base < Q4K_BLOCK_ELEMS ? cols - base : Q4K_BLOCK_ELEMS;
            memcpy(out + (size_t)r * (size_t)cols + base, tmp, (size_t)n * sizeof(float));
        }
    }
    return 0;
}

int ora_q4k_gemv_rows(const uint8_t *w, const float *x, float *y, int64_t n, int64_t k,
                      int64_t row_begin, int64_t row_end) {
    /* y[i] = sum_k W[i,k] * x[k] with W the row-wise Q4_K dequant and an f32
     * left-fold accumulator: reference_interpreter.zig:327-341 (tryFusedGemv,
     * linear tree shape), fed by doppler_rdrr_q4k.py:128-156. */
    if (n < 0 || k < 0 || row_begin < 0 || row_end > n || row_begin > row_end) return -1;
    int64_t nb = (k + Q4K_BLOCK_ELEMS - 1) / Q4K_BLOCK_ELEMS;
    float tmp[256];
    for (int64_t r = row_begin; r < row_end; ++r) {
        const uint8_t *row = w + (size_t)r * (size_t)nb * Q4K_BLOCK_BYTES;
        float acc = 0.0f;
        for (int64_t blk = 0; blk < nb; ++blk) {
            ora_q4k_dequant_block(row + blk * Q4K_BLOCK_BYTES, tmp);
            int64_t base = blk * Q4K_BLOCK_ELEMS;
            int64_t cnt = k - base < Q4K_BLOCK_ELEMS ? k - base : Q4K_BLOCK_ELEMS;
            for (int64_t i = 0; i < cnt; ++i) acc += tmp[i] * x[base + i];
        }
        y[r] = acc;
    }
    return 0;
}

int ora_q4k_gemv(const uint8_t *w, const float *x, float *y, int64_t n, int64_t k) {
    return ora_q4k_gemv_rows(w, x, y, n, k, 0, n);
}

static void q4k_row_dequant(const uint8_t *b, int64_t row, int64_t k, float *dst) {
    int64_t nb = (k + Q4K_BLOCK_ELEMS - 1) / Q4K_BLOCK_ELEMS;
    float tmp[256];
    const uint8_t *rowp = b + (size_t)row * (size_t)nb * Q4K_BLOCK_BYTES;
    for (int64_t blk = 0; blk < nb; ++blk) {
        ora_q4k_dequant_block(rowp + blk * Q4K_BLOCK_BYTES, tmp);
        int64_t base = blk * Q4K_BLOCK_ELEMS;
        int64_t cnt = k - base < Q4K_BLOCK_ELEMS ? k - base : Q4K_BLOCK_ELEMS;
        memcpy(dst + base, tmp, (size_t)cnt * sizeof(float));
    }
}

int ora_q4k_gemm_sampled(const uint16_t *a_bf16, const uint8_t *b, int64_t m, int64_t n,
                         int64_t k, const int64_t *mi, const int64_t *ni, int64_t count,
                         float *out) {
    /* C[m,n] = sum_k A[m,k] * dequant(B)[n,k] (emit_csl_matmul_q4k.zig:1-37:
     * B is row-major [N][K] Q4_K rows, A is [M][K]); bf16 A upcast exactly
     * (reference_interpreter.zig:2118-2124); f32 left-fold over k.
     * Evaluates only the listed (mi[t], ni[t]) entries. */
    if (m < 0 || n < 0 || k < 0 || count < 0) return -1;
    float *wrow = (float *)malloc((size_t)(k > 0 ? k : 1) * sizeof(float));
    if (!wrow) return -2;
    int64_t cached = -1;
    for (int64_t t = 0; t < count; ++t) {
        if (mi[t] < 0 || mi[t] >= m || ni[t] < 0 || ni[t] >= n) {
            free(wrow);
            return -1;
        }
        if (ni[t] != cached) {
            q4k_row_dequant(b, ni[t], k, wrow);
            cached = ni[t];
        }
        const uint16_t *arow = a_bf16 + (size_t)mi[t] * (size_t)k;
        float acc = 0.0f;
        for (int64_t kk = 0; kk < k; ++kk) acc += ora_bf16_to_f32(arow[kk]) * wrow[kk];
        out[t] = acc;
    }
    free(wrow);
    return 0;
}

int ora_q4k_gemm(const uint16_t *a_bf16, const uint8_t *b, float *c, int64_t m, int64_t n,
                 int64_t k) {
    if (m < 0 || n < 0 || k < 0) return -1;
    float *wrow = (float *)malloc((size_t)(k > 0 ? k : 1) * sizeof(float));
    if (!wrow) return -2;
    for (int64_t j = 0; j < n; ++j) {
        q4k_row_dequant(b, j, k, wrow);
        for (int64_t i = 0; i < m; ++i) {
            const uint16_t *ar = a_bf16 + (size_t)i * (size_t)k;
            float acc = 0.0f;
            for (int64_t kk = 0; kk < k; ++kk) acc += ora_bf16_to_f32(ar[kk]) * wrow[kk];
            c[(size_t)i * (size_t)n + j] = acc;
        }
    }
    free(wrow);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Dense GEMVs.                                                               */
/* ------------------------------------------------------------------------- */

int ora_f32_gemv(const float *w, const float *x, float *y, int64_t m, int64_t k) {
    /* reference_interpreter.zig:318-341 (linear tree shape, k == 0 -> 0). */
    if (m < 0 || k < 0) return -1;
    for (int64_t i = 0; i < m; ++i) {
        float acc = 0.0f;
        for (int64_t kk = 0; kk < k; ++kk) acc += w[(size_t)i * (size_t)k + kk] * x[kk];
        y[i] = acc;
    }
    return 0;
}

int ora_lm_head_gemv(const float *a, const uint16_t *b, float *c, int64_t m, int64_t n,
                     int64_t k, float alpha, int transpose_b) {
    /* lm_head_gemv.wgsl:79-168 (main; main_multicol :188-274 is the same
     * sum): C[col] = alpha * sum_k A[k] * f32(B(col, k)), B(col, k) =
     * B[col*K + k] when transpose_b == 1 (:105-116), B[k*N + col] otherwise
     * (:117-143).  The shader reads activation row 0 only; row r of a here
     * is computed the same way into row r of c.  Each sum is an f32
     * left-fold (reference_interpreter.zig:333-339) and alpha scales the
     * finished sum (:167). */
    if (m < 0 || n < 0 || k < 0 || (transpose_b != 0 && transpose_b != 1)) return -1;
    for (int64_t r = 0; r < m; ++r) {
        const float *ar = a + (size_t)r * (size_t)k;
        for (int64_t j = 0; j < n; ++j) {
            float acc = 0.0f;
            for (int64_t kk = 0; kk < k; ++kk) {
                const size_t at = transpose_b ? (size_t)j * (size_t)k + (size_t)kk
                                              : (size_t)kk * (size_t)n + (size_t)j;
                acc += ar[kk] * ora_f16_to_f32(b[at]);
            }
            c[(size_t)r * (size_t)n + j] = acc * alpha;
        }
    }
    return 0;
}

int ora_f16_gemv(const uint16_t *b, const float *a, float *c, int64_t n, int64_t k,
                 float alpha) {
    /* lm_head_gemv.wgsl:78-180 with transpose_b = 1 and one activation row. */
    return ora_lm_head_gemv(a, b, c, 1, n, k, alpha, 1);
}

int ora_int4g32_gemv(const uint32_t *q, const uint16_t *scales, const float *x, float *y,
                     int64_t m, int64_t n, int64_t k) {
    /* complex_fused_gemv_dequant.wgsl:18-23 (nibble idx%8 at bit 4*(idx%8),
     * value nib - 8) and :36-47 (scale [row][col / group], w * x); group 32,
     * f16 scales; m activation rows, each an f32 left-fold over k. */
    if (m < 0 || n < 0 || k < 0 || (k % 32) != 0) return -1;
    int64_t groups = k / 32;
    for (int64_t b = 0; b < m; ++b) {
        for (int64_t r = 0; r < n; ++r) {
            float acc = 0.0f;
            for (int64_t col = 0; col < k; ++col) {
                int64_t flat = r * k + col;
                uint32_t word = q[flat / 8];
                uint32_t nib = (word >> (4 * (uint32_t)(col % 8))) & 0xfu;
                float scale = ora_f16_to_f32(scales[r * groups + col / 32]);
                float wv = ((float)nib - 8.0f) * scale;
                acc += wv * x[b * k + col];
            }
            y[b * n + r] = acc;
        }
    }
    return 0;
}

int64_t ora_q8_0_element_count(int64_t bytes) {
    /* runtime/zig/src/doe_wgsl/csl_spec.zig:135-153: a zero size or one that
     * is not a whole number of 34-byte blocks is invalid; else 32 elements per
     * block. */
    if (bytes <= 0 || bytes % 34 != 0) return -1;
    return bytes / 34 * 32;
}

/* Weight (row, col) of row-wise Q8_0: block col / 32 of the row, whose bytes
 * are the f16 scale d (little-endian) then 32 int8 quants
 * (csl_spec.zig:121-125); weight = f32(q) * d. */
static float q8_0_weight(const uint8_t *w, int64_t row, int64_t col, int64_t nb) {
    const uint8_t *blk = w + (row * nb + col / 32) * 34;
    float d = ora_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    return (float)(int8_t)blk[2 + col % 32] * d;
}

int ora_q8_0_dequant(const uint8_t *w, float *out, int64_t n, int64_t k) {
    if (n < 0 || k < 0) return -1;
    int64_t nb = (k + 31) / 32;
    for (int64_t r = 0; r < n; ++r)
        for (int64_t c = 0; c < k; ++c) out[r * k + c] = q8_0_weight(w, r, c, nb);
    return 0;
}

int ora_q8_0_gemv(const uint8_t *w, const float *x, const float *residual, float *y, int64_t n,
                  int64_t k) {
    /* y[r] = f32 left-fold over k of weight * x, then + residual[r]: the
     * accumulation of ora_int4g32_gemv, so equal weights give equal sums. */
    if (n < 0 || k < 0) return -1;
    int64_t nb = (k + 31) / 32;
    for (int64_t r = 0; r < n; ++r) {
        float acc = 0.0f;
        for (int64_t c = 0; c < k; ++c) acc += q8_0_weight(w, r, c, nb) * x[c];
        y[r] = residual ? acc + residual[r] : acc;
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Normalisation and elementwise ops.                                         */
/* ------------------------------------------------------------------------- */

int ora_rmsnorm(const float *x, const float *w, float *out, int64_t rows, int64_t h,
                float eps, int weight_offset) {
    /* reference_interpreter.zig:510-526: f32 left-fold of x*x, mean = sum/H,
     * inv = 1/sqrt(mean + eps), out = x * inv * w.  weight_offset selects the
     * (1 + w) form of rmsnorm.wgsl:55-93 / run_csl_webgpu_emulator.mjs:509-526. */
    if (rows < 0 || h < 0) return -1;
    if (h == 0) return 0;
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + (size_t)r * (size_t)h;
        float *orow = out + (size_t)r * (size_t)h;
        float sum_sq = 0.0f;
        for (int64_t i = 0; i < h; ++i) sum_sq += xr[i] * xr[i];
        float mean_sq = sum_sq / (float)h;
        float inv_rms = 1.0f / sqrtf(mean_sq + eps);
        for (int64_t i = 0; i < h; ++i) {
            float scale = weight_offset ? 1.0f + w[i] : w[i];
            orow[i] = xr[i] * inv_rms * scale;
        }
    }
    return 0;
}

int ora_rope_table(float *freq_cis, int64_t max_pos, int64_t head_dim, double base) {
    /* freq_cis[(pos*half + i)*2 + {0,1}] = {cos, sin}(pos * base^(-2i/D)), the
     * table layout rope.wgsl:27-29 reads.  The reference builds it on the host
     * outside this tree; here the angle is computed in double and cos/sin
     * are rounded once to f32. */
    if (max_pos < 0 || head_dim <= 0 || (head_dim % 2) != 0) return -1;
    int64_t half = head_dim / 2;
    for (int64_t p = 0; p < max_pos; ++p) {
        for (int64_t i = 0; i < half; ++i) {
            double inv_freq = pow(base, -2.0 * (double)i / (double)head_dim);
            double ang = (double)p * inv_freq;
            freq_cis[(p * half + i) * 2 + 0] = (float)cos(ang);
            freq_cis[(p * half + i) * 2 + 1] = (float)sin(ang);
        }
    }
    return 0;
}

int ora_rope(float *qk, const float *freq_cis, int64_t seq_len, int64_t num_heads,
             int64_t head_dim, int64_t position_offset) {
    /* rope.wgsl:12-35: rotate-half pairs (i, i + D/2) of qk[seq][head][dim],
     * angle row pos = seq + position_offset. */
    if (seq_len < 0 || num_heads < 0 || head_dim <= 0 || (head_dim % 2) != 0) return -1;
    int64_t half = head_dim / 2;
    for (int64_t s = 0; s < seq_len; ++s) {
        int64_t pos = s + position_offset;
        for (int64_t h = 0; h < num_heads; ++h) {
            float *base = qk + (size_t)((s * num_heads + h) * head_dim);
            for (int64_t i = 0; i < half; ++i) {
                float x0 = base[i], x1 = base[i + half];
                float c = freq_cis[(pos * half + i) * 2], sn = freq_cis[(pos * half + i) * 2 + 1];
                base[i] = x0 * c - x1 * sn;
                base[i + half] = x0 * sn + x1 * c;
            }
        }
    }
    return 0;
}

int ora_rope_pairs(float *x, const float *cos_t, const float *sin_t, int64_t head_dim,
                   int64_t num_pairs, int interleaved) {
    /* run_csl_webgpu_emulator.mjs:589-613 for one head: interleaved pairs
     * (2i, 2i+1) or split pairs (i, i + num_pairs). */
    if (head_dim <= 0 || num_pairs < 0 || 2 * num_pairs > head_dim) return -1;
    for (int64_t p = 0; p < num_pairs; ++p) {
        int64_t d0 = interleaved ? 2 * p : p;
        int64_t d1 = interleaved ? d0 + 1 : d0 + num_pairs;
        float x0 = x[d0], x1 = x[d1];
        x[d0] = x0 * cos_t[p] - x1 * sin_t[p];
        x[d1] = x0 * sin_t[p] + x1 * cos_t[p];
    }
    return 0;
}

int ora_geglu(const float *gate, const float *up, float *out, int64_t n) {
    /* reference_interpreter.zig:1027-1045 (gelu arm of tryGated) and
     * gelu_gated.wgsl:5-14: inner = a*(x + b*x*x*x) clamped to [-15, 15],
     * act = 0.5*x*(1 + tanh(inner)), out = act * up. */
    if (n < 0) return -1;
    const float ga = 0.7978845608028654f;
    const float gb = 0.044715f;
    for (int64_t i = 0; i < n; ++i) {
        float x = gate[i];
        float inner = ga * (x + gb * x * x * x);
        if (inner < -15.0f) inner = -15.0f;
        if (inner > 15.0f) inner = 15.0f;
        float act = 0.5f * x * (1.0f + tanhf(inner));
        out[i] = act * up[i];
    }
    return 0;
}

int ora_gated(const float *gate, const float *input, float *out, int64_t n, int kind) {
    /* reference_interpreter.zig:1023-1052 (tryGated): act(gate) * input with
     *   kind 0 gelu    : inner = a*(x + b*x^3) clamped to [-15, 15],
     *                    0.5*x*(1 + tanh(inner))
     *   kind 1 silu    : x / (1 + exp(z)),  z = clamp(-x, -15, 15)
     *   kind 2 sigmoid : 1 / (1 + exp(z)),  z = clamp(-x, -15, 15)
     * all in f32 (the platform expf / tanhf). */
    if (n < 0 || kind < 0 || kind > 2) return -1;
    const float ga = 0.7978845608028654f;
    const float gb = 0.044715f;
    for (int64_t i = 0; i < n; ++i) {
        float x = gate[i];
        float act;
        if (kind == 0) {
            float inner = ga * (x + gb * x * x * x);
            if (inner < -15.0f) inner = -15.0f;
            if (inner > 15.0f) inner = 15.0f;
            act = 0.5f * x * (1.0f + tanhf(inner));
        } else {
            float z = -x;
            if (z < -15.0f) z = -15.0f;
            if (z > 15.0f) z = 15.0f;
            act = (kind == 1 ? x : 1.0f) / (1.0f + expf(z));
        }
        out[i] = act * input[i];
    }
    return 0;
}

int ora_l2_normalize(const float *in, float *out, int64_t rows, int64_t hidden, float eps) {
    /* reference_interpreter.zig:1284-1361 (tryL2Normalize), per row:
     * sq = f32 left-fold of x*x, inv = 1 / sqrt(sq + eps), out = x * inv. */
    if (rows < 0 || hidden <= 0) return -1;
    for (int64_t r = 0; r < rows; ++r) {
        const float *x = in + r * hidden;
        float sq = 0.0f;
        for (int64_t d = 0; d < hidden; ++d) sq += x[d] * x[d];
        float inv = 1.0f / sqrtf(sq + eps);
        for (int64_t d = 0; d < hidden; ++d) out[r * hidden + d] = x[d] * inv;
    }
    return 0;
}

int ora_conv1d_depthwise(const float *in, const float *w, const float *bias, float *out, int64_t tokens,
                         int64_t channels, int64_t kernel_size) {
    /* reference_interpreter.zig:1363-1455 (tryConv1DDepthwise): input and
     * output [token][channel], weight [channel][kernel_size], causal:
     * out[t][c] = bias[c] + sum_{k, t - (K-1-k) >= 0} in[t-(K-1-k)][c] w[c][k],
     * the terms in k order from the bias (or 0). */
    if (tokens < 0 || channels <= 0 || kernel_size <= 0) return -1;
    for (int64_t t = 0; t < tokens; ++t) {
        for (int64_t c = 0; c < channels; ++c) {
            float acc = bias ? bias[c] : 0.0f;
            for (int64_t k = 0; k < kernel_size; ++k) {
                int64_t ti = t - (kernel_size - 1 - k);
                if (ti < 0) continue;
                acc += in[ti * channels + c] * w[c * kernel_size + k];
            }
            out[t * channels + c] = acc;
        }
    }
    return 0;
}

int ora_linear_attention(const float *q, const float *k, const float *v, const float *gate, float *state,
                         float *out, int64_t tokens, int64_t heads, int64_t key_dim, int64_t value_dim,
                         const float *a_log) {
    /* reference_interpreter.zig:1457-1596 (tryLinearAttention; the gated
     * DeltaNet single-query shared-norm form of
     * emit_kernel_body_linear_attention.zig), per token and head, with
     * alpha = 1 - exp(-A_log) (A_log = 0.5 when a_log is NULL, the
     * interpreter's fixed value) and decay = 1 - alpha:
     *   for d: dot = sum_k S[d][k] kin[k]            (f32 left-fold)
     *          S[d][k] = decay * S[d][k] + (alpha * (q[d] - dot)) * kin[k]
     *   out[d] = sum_k S[d][k] v[k] + sigmoid(g[d]) * q[d]
     * q, gate, out [token][head][value_dim]; k, v [token][head][key_dim];
     * state [head][value_dim][key_dim], updated in place token after token. */
    if (tokens < 0 || heads <= 0 || key_dim <= 0 || value_dim <= 0) return -1;
    for (int64_t t = 0; t < tokens; ++t) {
        for (int64_t h = 0; h < heads; ++h) {
            const float al = a_log ? a_log[h] : 0.5f;
            const float alpha = 1.0f - expf(-al);
            const float decay = 1.0f - alpha;
            const float *qh = q + (t * heads + h) * value_dim;
            const float *gh = gate + (t * heads + h) * value_dim;
            const float *kh = k + (t * heads + h) * key_dim;
            const float *vh = v + (t * heads + h) * key_dim;
            float *S = state + h * value_dim * key_dim;
            for (int64_t d = 0; d < value_dim; ++d) {
                float dot = 0.0f;
                for (int64_t j = 0; j < key_dim; ++j) dot += S[d * key_dim + j] * kh[j];
                const float scaled = alpha * (qh[d] - dot);
                for (int64_t j = 0; j < key_dim; ++j)
                    S[d * key_dim + j] = decay * S[d * key_dim + j] + scaled * kh[j];
            }
            float *oh = out + (t * heads + h) * value_dim;
            for (int64_t d = 0; d < value_dim; ++d) {
                float acc = 0.0f;
                for (int64_t j = 0; j < key_dim; ++j) acc += S[d * key_dim + j] * vh[j];
                const float sg = 1.0f / (1.0f + expf(-gh[d]));
                oh[d] = acc + sg * qh[d];
            }
        }
    }
    return 0;
}

int ora_residual(const float *a, const float *b, float *out, int64_t n) {
    /* run_csl_webgpu_emulator.mjs:482-489. */
    if (n < 0) return -1;
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
    return 0;
}

int64_t ora_argmax(const float *logits, int64_t n) {
    /* run_csl_webgpu_emulator.mjs:841-878 with softcap 0 and temperature 1:
     * strict '>' scan from -FLT_MAX, so the lowest index wins a tie. */
    if (n <= 0) return -1;
    float best = -FLT_MAX;
    int64_t idx = 0;
    for (int64_t i = 0; i < n; ++i) {
        if (logits[i] > best) {
            best = logits[i];
            idx = i;
        }
    }
    return idx;
}

int ora_embed_gather(const uint16_t *table_f16, const int32_t *ids, float *out,
                     int64_t n_ids, int64_t vocab, int64_t hidden, float scale) {
    /* run_csl_webgpu_emulator.mjs:528-551: out[t] = table[id[t]], ids outside
     * the table give zeros.  scale multiplies each row (1.0 for a plain gather). */
    if (n_ids < 0 || vocab < 0 || hidden < 0) return -1;
    for (int64_t t = 0; t < n_ids; ++t) {
        int64_t id = ids[t];
        for (int64_t d = 0; d < hidden; ++d) {
            out[t * hidden + d] = (id >= 0 && id < vocab)
                                      ? ora_f16_to_f32(table_f16[id * hidden + d]) * scale
                                      : 0.0f;
        }
    }
    return 0;
}

int ora_gather_f32(const uint32_t *ids, const float *table, float *out, int64_t n_ids,
                   int64_t vocab, int64_t hidden) {
    /* reference_interpreter.zig:4143-4219 (gather: out[t][h] = table[ids[t]][h],
     * u32 indices, f32 table) and :4221-4276 (an index outside the table
     * rejects the whole run, nothing is clamped): returns -2 then, with out
     * untouched. */
    if (n_ids < 0 || vocab < 0 || hidden < 0) return -1;
    for (int64_t t = 0; t < n_ids; ++t)
        if ((int64_t)ids[t] >= vocab) return -2;
    for (int64_t t = 0; t < n_ids; ++t)
        for (int64_t h = 0; h < hidden; ++h)
            out[t * hidden + h] = table[(int64_t)ids[t] * hidden + h];
    return 0;
}

int ora_kv_write(const float *k_proj, const float *v_proj, uint16_t *k_cache,
                 uint16_t *v_cache, int64_t num_kv_heads, int64_t max_seq, int64_t head_dim,
                 int64_t pos, int kv_layout) {
    /* run_csl_webgpu_emulator.mjs:615-644: cache[h][pos][:] = proj[h][:],
     * pos >= max_seq is an error; the f16 cache stores RNE-rounded values. */
    if (num_kv_heads < 0 || head_dim < 0 || pos < 0 || pos >= max_seq) return -1;
    for (int64_t h = 0; h < num_kv_heads; ++h) {
        size_t dst = kv_layout == 0 ? (size_t)((h * max_seq + pos) * head_dim)
                                    : (size_t)((pos * num_kv_heads + h) * head_dim);
        for (int64_t d = 0; d < head_dim; ++d) {
            k_cache[dst + d] = ora_f32_to_f16(k_proj[h * head_dim + d]);
            v_cache[dst + d] = ora_f32_to_f16(v_proj[h * head_dim + d]);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Attention.                                                                 */
/* ------------------------------------------------------------------------- */

static size_t kv_index(int kv_layout, int64_t kvh, int64_t pos, int64_t num_kv_heads,
                       int64_t kv_stride, int64_t head_dim) {
    return kv_layout == 0 ? (size_t)((kvh * kv_stride + pos) * head_dim)
                          : (size_t)((pos * num_kv_heads + kvh) * head_dim);
}

int ora_attn_decode(const float *q, const uint16_t *k, const uint16_t *v, float *o,
                    int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                    int64_t kv_len, int64_t kv_stride, float scale, float softcap,
                    int64_t sliding_window, int kv_layout) {
    /* Two-pass stable softmax in f32 per reference_interpreter.zig:1175-1265
     * (scores, max, exp-sum, O = sum v * (w / sum)), with the GQA head map
     * kv = h / (Hq / Hkv) (attention_head256_f16kv.wgsl:46-49), the decode
     * query at position kv_len - 1, the sliding window of :122-127 and the
     * softcap of :197-199.  K/V are f16, upcast exactly. */
    if (num_heads <= 0 || num_kv_heads <= 0 || (num_heads % num_kv_heads) != 0 ||
        head_dim <= 0 || kv_len <= 0 || (kv_layout == 0 && kv_stride < kv_len))
        return -1;
    int64_t group = num_heads / num_kv_heads;
    int64_t min_key = 0;
    if (sliding_window > 0 && kv_len - 1 >= sliding_window) min_key = kv_len - sliding_window;
    float *scores = (float *)malloc((size_t)kv_len * sizeof(float));
    if (!scores) return -2;
    for (int64_t h = 0; h < num_heads; ++h) {
        int64_t kvh = h / group;
        const float *qh = q + h * head_dim;
        float max_score = -INFINITY;
        for (int64_t t = min_key; t < kv_len; ++t) {
            const uint16_t *kr = k + kv_index(kv_layout, kvh, t, num_kv_heads, kv_stride, head_dim);
            float dot = 0.0f;
            for (int64_t d = 0; d < head_dim; ++d) dot += qh[d] * ora_f16_to_f32(kr[d]);
            float s = dot * scale;
            if (softcap > 0.0f) s = tanhf(s / softcap) * softcap;
            scores[t] = s;
            if (s > max_score) max_score = s;
        }
        float sum_exp = 0.0f;
        for (int64_t t = min_key; t < kv_len; ++t) {
            float e = expf(scores[t] - max_score);
            scores[t] = e;
            sum_exp += e;
        }
        for (int64_t d = 0; d < head_dim; ++d) {
            float acc = 0.0f;
            for (int64_t t = min_key; t < kv_len; ++t) {
                const uint16_t *vr =
                    v + kv_index(kv_layout, kvh, t, num_kv_heads, kv_stride, head_dim);
                acc += ora_f16_to_f32(vr[d]) * (scores[t] / sum_exp);
            }
            o[h * head_dim + d] = acc;
        }
    }
    free(scores);
    return 0;
}

int ora_attn_prefill(const float *q, const float *k, const float *v, float *o,
                     int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                     int64_t q_len, int64_t kv_len, int64_t start_pos, float scale,
                     int causal, int64_t row_begin, int64_t row_end) {
    /* Causal multi-query attention, one two-pass f32 softmax per (query,
     * head) as in ora_attn_decode.  q/o are [q_len][num_heads][head_dim]
     * (attention_head256_f16kv.wgsl:94-96, :258), k/v are
     * [num_kv_heads][kv_len][head_dim]; query i sits at absolute position
     * start_pos + i and, when causal, sees keys 0..start_pos + i
     * (attention_head256_f16kv.wgsl:115-121 with kv_start 0).  Only query rows
     * [row_begin, row_end) are evaluated. */
    if (num_heads <= 0 || num_kv_heads <= 0 || (num_heads % num_kv_heads) != 0 ||
        head_dim <= 0 || q_len < 0 || kv_len <= 0 || row_begin < 0 || row_end > q_len ||
        row_begin > row_end)
        return -1;
    int64_t group = num_heads / num_kv_heads;
    float *scores = (float *)malloc((size_t)kv_len * sizeof(float));
    if (!scores) return -2;
    for (int64_t i = row_begin; i < row_end; ++i) {
        int64_t limit = kv_len;
        if (causal) {
            int64_t lim = start_pos + i + 1;
            limit = lim < kv_len ? lim : kv_len;
        }
        for (int64_t h = 0; h < num_heads; ++h) {
            int64_t kvh = h / group;
            const float *qh = q + (size_t)((i * num_heads + h) * head_dim);
            float *oh = o + (size_t)((i * num_heads + h) * head_dim);
            if (limit <= 0) {
                for (int64_t d = 0; d < head_dim; ++d) oh[d] = 0.0f;
                continue;
            }
            float max_score = -INFINITY;
            for (int64_t t = 0; t < limit; ++t) {
                const float *kr = k + (size_t)((kvh * kv_len + t) * head_dim);
                float dot = 0.0f;
                for (int64_t d = 0; d < head_dim; ++d) dot += qh[d] * kr[d];
                float s = dot * scale;
                scores[t] = s;
                if (s > max_score) max_score = s;
            }
            float sum_exp = 0.0f;
            for (int64_t t = 0; t < limit; ++t) {
                float e = expf(scores[t] - max_score);
                scores[t] = e;
                sum_exp += e;
            }
            for (int64_t d = 0; d < head_dim; ++d) {
                float acc = 0.0f;
                for (int64_t t = 0; t < limit; ++t)
                    acc += v[(size_t)((kvh * kv_len + t) * head_dim + d)] * (scores[t] / sum_exp);
                oh[d] = acc;
            }
        }
    }
    free(scores);
    return 0;
}
