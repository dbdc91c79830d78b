/*
 * gaje_oracle.c — CPU restatement of the GAJE quantised decode kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle and the CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only as the checker (or as the timed CPU baseline);
 * the product library never links or calls it.
 *
 * Every function restates one reference function (file:line cited on each),
 * using the same x86 intrinsic sequence and the same scalar operation order,
 * so that on an AVX2+FMA+F16C host its results are bit-identical to the Rust
 * AVX2 path.  Assumptions that only a Rust build could confirm (and which are
 * therefore stated, not verified):
 *   - `is_x86_feature_detected!("avx2") && ("fma")` selects the AVX2 branches
 *     (orc_init() refuses to run on a host without AVX2/FMA/F16C);
 *   - LLVM does not reassociate the scalar loops of attention.rs:104-117;
 *   - f32::exp / powf / sin_cos lower to glibc expf / powf / sinf / cosf.
 * Compile with -ffp-contract=off: Rust never contracts a*b+c into an FMA.
 *
 * Parity status (what pins each function) is listed in oracle/oracle.py.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define Q4_0_BLOCK_BYTES 20 /* repr(C, packed) {f16 scale, f16 min, u8 qs[16]} */
#define Q8_0_BLOCK_BYTES 34 /* repr(C, packed) {f16 scale, i8 qs[32]} (blocks.rs:36-41) */

/* The exponential of attention.rs:106 and activation.rs:42-44 (f32::exp ->
 * the C library's expf); overridable only to study sensitivity. */
#ifndef ORC_EXPF
#define ORC_EXPF expf
#endif

static inline float h2f(uint16_t h) { return _cvtsh_ss(h); }

/* Host capability check: the restatement is only the reference's x86 path
 * when AVX2 and FMA are present (genomic.rs:215-220, dot.rs:46, norm.rs:54). */
int orc_init(void) {
    __builtin_cpu_init();
    if (!__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("fma") ||
        !__builtin_cpu_supports("f16c"))
        return -1;
    return 0;
}

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int orc_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* half::f16::to_f32 / from_f32 (half 2.4.1): exact widening, RNE narrowing. */
float orc_f16_to_f32(uint16_t h) { return h2f(h); }
uint16_t orc_f32_to_f16(float f) { return _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }

/* f32::exp as the reference calls it (attention.rs:106, activation.rs:42-44). */
void orc_expf_batch(const float *x, float *y, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) y[i] = ORC_EXPF(x[i]);
}

/* Q4_0Block::dequantize_weight — src/io/header/blocks.rs:18-30.
 * Even index = low nibble; w = f32(q)*scale + min as a mul then an add. */
float orc_q4_0_dequant_weight(const uint8_t *block, int idx) {
    uint16_t hs, hm;
    memcpy(&hs, block, 2);
    memcpy(&hm, block + 2, 2);
    uint8_t byte = block[4 + idx / 2];
    uint8_t q = (idx % 2 == 0) ? (byte & 0x0F) : (byte >> 4);
    float scale = h2f(hs), mn = h2f(hm);
    float prod = (float)q * scale;
    return prod + mn;
}

/* Row dequantisation as GenomicLinear::get_row_core does it for the Q4_0
 * variant (src/nn/linear/forward.rs:260-270): block b fills out[32b..32b+32). */
void orc_q4_0_dequant(const uint8_t *blocks, size_t nblocks, float *out) {
    for (size_t b = 0; b < nblocks; b++)
        for (int k = 0; k < 32; k++)
            out[b * 32 + k] = orc_q4_0_dequant_weight(blocks + b * Q4_0_BLOCK_BYTES, k);
}

/* genomic_dot_product_q4_0_avx2 — src/compute/kernels/genomic.rs:263-336. */
float orc_dot_q4_0_avx2(const uint8_t *blocks, const float *input, size_t n_blocks) {
    __m256 acc = _mm256_setzero_ps();
    const __m128i mask_low = _mm_set1_epi8(0x0F);
    for (size_t j = 0; j < n_blocks; j++) {
        const uint8_t *blk = blocks + j * Q4_0_BLOCK_BYTES;
        uint16_t hs, hm;
        memcpy(&hs, blk, 2);
        memcpy(&hm, blk + 2, 2);
        const __m256 v_scale = _mm256_set1_ps(h2f(hs));
        const __m256 v_min = _mm256_set1_ps(h2f(hm));
        const float *in = input + j * 32;
        __m128i v_qs = _mm_loadu_si128((const __m128i *)(blk + 4));
        __m128i low = _mm_and_si128(v_qs, mask_low);
        __m128i high = _mm_and_si128(_mm_srli_epi16(v_qs, 4), mask_low);
        __m128i il_lo = _mm_unpacklo_epi8(low, high);
        __m128i il_hi = _mm_unpackhi_epi8(low, high);

        __m256 q = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(il_lo));
        __m256 d = _mm256_fmadd_ps(q, v_scale, v_min);
        acc = _mm256_fmadd_ps(d, _mm256_loadu_ps(in), acc);

        q = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(il_lo, 8)));
        d = _mm256_fmadd_ps(q, v_scale, v_min);
        acc = _mm256_fmadd_ps(d, _mm256_loadu_ps(in + 8), acc);

        q = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(il_hi));
        d = _mm256_fmadd_ps(q, v_scale, v_min);
        acc = _mm256_fmadd_ps(d, _mm256_loadu_ps(in + 16), acc);

        q = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(il_hi, 8)));
        d = _mm256_fmadd_ps(q, v_scale, v_min);
        acc = _mm256_fmadd_ps(d, _mm256_loadu_ps(in + 24), acc);
    }
    __m128 vlow = _mm256_castps256_ps128(acc);
    __m128 vhigh = _mm256_extractf128_ps(acc, 1);
    __m128 v128 = _mm_add_ps(vlow, vhigh);
    __m128 hi = _mm_movehl_ps(v128, v128);
    __m128 sum = _mm_add_ps(v128, hi);
    __m128 shuf = _mm_shuffle_ps(sum, sum, 1);
    __m128 fin = _mm_add_ss(sum, shuf);
    float total = _mm_cvtss_f32(fin);
    return fabsf(total) < 1e-6f ? 0.0f : total;
}

/* Q8_0Block::dequantize_weight — src/io/header/blocks.rs:43-49: f32(q) * scale. */
float orc_q8_0_dequant_weight(const uint8_t *block, int idx) {
    uint16_t hs;
    memcpy(&hs, block, 2);
    float q = (float)(int8_t)block[2 + idx];
    return q * h2f(hs);
}

void orc_q8_0_dequant(const uint8_t *blocks, size_t nblocks, float *out) {
    for (size_t b = 0; b < nblocks; b++)
        for (int k = 0; k < 32; k++)
            out[b * 32 + k] = orc_q8_0_dequant_weight(blocks + b * Q8_0_BLOCK_BYTES, k);
}

/* genomic_dot_product_q8_0_avx2 — src/compute/kernels/genomic.rs:377-448:
 * per block, the 32 signed codes widened to four 8-float vectors (elements
 * 8c..8c+7), dq = q * scale, acc = fma(dq, x, acc) in c order; the horizontal
 * sum and the 1e-6 flush of the Q4_0 kernel. */
float orc_dot_q8_0_avx2(const uint8_t *blocks, const float *input, size_t n_blocks) {
    __m256 acc = _mm256_setzero_ps();
    for (size_t j = 0; j < n_blocks; j++) {
        const uint8_t *blk = blocks + j * Q8_0_BLOCK_BYTES;
        uint16_t hs;
        memcpy(&hs, blk, 2);
        const __m256 v_scale = _mm256_set1_ps(h2f(hs));
        const __m256i v_qs = _mm256_loadu_si256((const __m256i *)(blk + 2));
        const __m128i lo_128 = _mm256_castsi256_si128(v_qs);
        const __m128i hi_128 = _mm256_extracti128_si256(v_qs, 1);
        const __m128i lo_lo_16 = _mm_cvtepi8_epi16(lo_128);
        const __m128i lo_hi_16 = _mm_cvtepi8_epi16(_mm_srli_si128(lo_128, 8));
        const __m256 q_0 = _mm256_cvtepi32_ps(_mm256_cvtepi16_epi32(lo_lo_16));
        const __m256 q_1 = _mm256_cvtepi32_ps(_mm256_cvtepi16_epi32(lo_hi_16));
        const __m128i hi_lo_16 = _mm_cvtepi8_epi16(hi_128);
        const __m128i hi_hi_16 = _mm_cvtepi8_epi16(_mm_srli_si128(hi_128, 8));
        const __m256 q_2 = _mm256_cvtepi32_ps(_mm256_cvtepi16_epi32(hi_lo_16));
        const __m256 q_3 = _mm256_cvtepi32_ps(_mm256_cvtepi16_epi32(hi_hi_16));
        const float *in = input + j * 32;
        const __m256 x_0 = _mm256_loadu_ps(in), x_1 = _mm256_loadu_ps(in + 8);
        const __m256 x_2 = _mm256_loadu_ps(in + 16), x_3 = _mm256_loadu_ps(in + 24);
        acc = _mm256_fmadd_ps(_mm256_mul_ps(q_0, v_scale), x_0, acc);
        acc = _mm256_fmadd_ps(_mm256_mul_ps(q_1, v_scale), x_1, acc);
        acc = _mm256_fmadd_ps(_mm256_mul_ps(q_2, v_scale), x_2, acc);
        acc = _mm256_fmadd_ps(_mm256_mul_ps(q_3, v_scale), x_3, acc);
    }
    __m128 vlow = _mm256_castps256_ps128(acc);
    __m128 vhigh = _mm256_extractf128_ps(acc, 1);
    __m128 v128 = _mm_add_ps(vlow, vhigh);
    __m128 hi = _mm_movehl_ps(v128, v128);
    __m128 sum = _mm_add_ps(v128, hi);
    __m128 shuf = _mm_shuffle_ps(sum, sum, 1);
    __m128 fin = _mm_add_ss(sum, shuf);
    float total = _mm_cvtss_f32(fin);
    return fabsf(total) < 1e-6f ? 0.0f : total;
}

/* Scalar fallback of genomic_dot_product_q8_0 — genomic.rs:338-372: per block
 * sum(q * x) in element order, times the scale.  Not the path an AVX2 host takes;
 * kept for the factored-form check. */
float orc_dot_q8_0_scalar(const uint8_t *blocks, const float *input, size_t n_blocks) {
    float total = 0.0f;
    for (size_t j = 0; j < n_blocks; j++) {
        const uint8_t *blk = blocks + j * Q8_0_BLOCK_BYTES;
        uint16_t hs;
        memcpy(&hs, blk, 2);
        float s = 0.0f;
        for (int k = 0; k < 32; k++) {
            float p = (float)(int8_t)blk[2 + k] * input[j * 32 + k];
            s += p;
        }
        float t = s * h2f(hs);
        total += t;
    }
    return fabsf(total) < 1e-6f ? 0.0f : total;
}

/* quantize_q8_0_native's block loop — src/compute/quantize/python.rs:235-300:
 * scale = max|w| / 127, inv = 1/scale when scale > 1e-7 (else every q = 0),
 * q = round(w * inv) (half away from zero) clamped to [-128, 127], the scale
 * stored as f16 (round to nearest even). */
void orc_q8_0_quantize(const float *w, size_t nblocks, uint8_t *out) {
    for (size_t b = 0; b < nblocks; b++) {
        const float *blk = w + b * 32;
        uint8_t *o = out + b * Q8_0_BLOCK_BYTES;
        float max_abs = 0.0f;
        for (int k = 0; k < 32; k++) {
            float a = fabsf(blk[k]);
            if (a > max_abs) max_abs = a;
        }
        float scale = max_abs / 127.0f;
        float inv = scale > 1e-7f ? 1.0f / scale : 0.0f;
        for (int k = 0; k < 32; k++) {
            int8_t q = 0;
            if (scale > 1e-7f) {
                float r = roundf(blk[k] * inv);
                if (r < -128.0f) r = -128.0f;
                if (r > 127.0f) r = 127.0f;
                q = (int8_t)r;
            }
            o[2 + k] = (uint8_t)q;
        }
        uint16_t hs = orc_f32_to_f16(scale);
        memcpy(o, &hs, 2);
    }
}

/* Scalar fallback of genomic_dot_product_q4_0 — genomic.rs:227-260.  Not the
 * path the reference takes on an AVX2 host; kept for the factored-form check. */
float orc_dot_q4_0_scalar(const uint8_t *blocks, const float *input, size_t n_blocks) {
    float total_sum = 0.0f;
    for (size_t j = 0; j < n_blocks; j++) {
        const uint8_t *blk = blocks + j * Q4_0_BLOCK_BYTES;
        uint16_t hs, hm;
        memcpy(&hs, blk, 2);
        memcpy(&hm, blk + 2, 2);
        float scale = h2f(hs), mn = h2f(hm);
        const float *in = input + j * 32;
        float sum_q_in = 0.0f, sum_in = 0.0f;
        for (int k = 0; k < 16; k++) {
            uint8_t byte = blk[4 + k];
            float q0 = (float)(byte & 0x0F), q1 = (float)(byte >> 4);
            float x0 = in[k * 2], x1 = in[k * 2 + 1];
            float a = q0 * x0, b = q1 * x1;
            sum_q_in += a + b;
            sum_in += x0 + x1;
        }
        float s1 = sum_q_in * scale, s2 = sum_in * mn;
        total_sum += s1 + s2;
    }
    return fabsf(total_sum) < 1e-6f ? 0.0f : total_sum;
}

/* genomic_dot_product_4bit (LUT layout, high nibble = even element) —
 * genomic.rs:148-204.  Four scalar accumulators in the :177-185 pattern. */
float orc_dot_4bit(const uint8_t *weights, const float *input, const float *centroids,
                   size_t stride_4bit, size_t n_blocks) {
    size_t block_size = stride_4bit * 2;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    for (size_t j = 0; j < n_blocks; j++) {
        const float *in = input + j * block_size;
        const uint8_t *w = weights + j * stride_4bit;
        const float *c = centroids + j * 16;
        size_t k = 0;
        while (k + 4 <= stride_4bit) {
            uint8_t b0 = w[k], b1 = w[k + 1], b2 = w[k + 2], b3 = w[k + 3];
            const float *ip = in + k * 2;
            s0 += c[b0 >> 4] * ip[0];
            s1 += c[b0 & 0x0F] * ip[1];
            s2 += c[b1 >> 4] * ip[2];
            s3 += c[b1 & 0x0F] * ip[3];
            s0 += c[b2 >> 4] * ip[4];
            s1 += c[b2 & 0x0F] * ip[5];
            s2 += c[b3 >> 4] * ip[6];
            s3 += c[b3 & 0x0F] * ip[7];
            k += 4;
        }
        while (k < stride_4bit) {
            uint8_t byte = w[k];
            s0 += c[byte >> 4] * in[k * 2];
            s1 += c[byte & 0x0F] * in[k * 2 + 1];
            k += 1;
        }
    }
    float total = s0 + s1 + s2 + s3;
    return fabsf(total) < 1e-6f ? 0.0f : total;
}

/* genomic_dot_product (2-bit, Gray-coded centroids) — genomic.rs:17-144.  The
 * reference forces genomic_dot_product_scalar (:26), whose x86 AVX2+FMA branch
 * (:67-122) runs per block: codes are read MSB first, code 00/01/10/11 selects
 * c0/c1/c3/c2 of the block's four centroids times the modulation factors
 * (:60-70); 4-byte steps feed 16 weights to two 8-lane FMA accumulators
 * (weights 0-7 of the step to the first, 8-15 to the second), the lanes are
 * summed pairwise and reduced as ((a0+a4)+(a1+a5))+((a2+a6)+(a3+a7)), and
 * that block value is added to the row sum.  Bytes past the last 4-byte step
 * go through the scalar loop (:124-133), each product rounded and added to the
 * row sum.  |sum| < 1e-5 flushes to 0 (:137-139).  centroids advance by 4 per
 * block from the row's base; modulation may be NULL (all 1). */
float orc_dot_2bit(const uint8_t *weights, const float *input, const float *centroids, size_t stride,
                   size_t n_blocks, const float *modulation) {
    static const float one[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    const float *m = modulation ? modulation : one;
    float sum = 0.0f;
    for (size_t j = 0; j < n_blocks; j++) {
        const float *in = input + j * stride * 4;
        const uint8_t *w = weights + j * stride;
        const float *cp = centroids + j * 4;
        const float c0 = cp[0] * m[0], c1 = cp[1] * m[1], c2 = cp[2] * m[2], c3 = cp[3] * m[3];
        const float ca[4] = {c0, c1, c3, c2};
        float acc0[8] = {0}, acc1[8] = {0};
        size_t k = 0;
        while (k + 4 <= stride) {
            float wv[16];
            for (int q = 0; q < 4; q++)
                for (int b = 0; b < 4; b++) wv[4 * q + b] = ca[(w[k + q] >> (6 - 2 * b)) & 3];
            for (int e = 0; e < 8; e++) {
                acc0[e] = fmaf(wv[e], in[k * 4 + e], acc0[e]);
                acc1[e] = fmaf(wv[8 + e], in[k * 4 + 8 + e], acc1[e]);
            }
            k += 4;
        }
        float a[8];
        for (int e = 0; e < 8; e++) a[e] = acc0[e] + acc1[e];
        const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
        const float r = (s0 + s1) + (s2 + s3);
        sum += r;
        while (k < stride) {
            const uint8_t byte = w[k];
            for (int b = 0; b < 4; b++) {
                const float p = ca[(byte >> ((3 - b) * 2)) & 3] * in[k * 4 + b];
                sum += p;
            }
            k += 1;
        }
    }
    return fabsf(sum) < 1e-5f ? 0.0f : sum;
}

/* The same function without the AVX2 branch (a host lacking AVX2/FMA runs
 * only the scalar loop, :124-133): one rounded product and one add per weight. */
float orc_dot_2bit_scalar(const uint8_t *weights, const float *input, const float *centroids, size_t stride,
                          size_t n_blocks, const float *modulation) {
    static const float one[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    const float *m = modulation ? modulation : one;
    float sum = 0.0f;
    for (size_t j = 0; j < n_blocks; j++) {
        const float *cp = centroids + j * 4;
        const float ca[4] = {cp[0] * m[0], cp[1] * m[1], cp[3] * m[3], cp[2] * m[2]};
        for (size_t k = 0; k < stride; k++) {
            const uint8_t byte = weights[j * stride + k];
            for (int b = 0; b < 4; b++) {
                const float p = ca[(byte >> ((3 - b) * 2)) & 3] * input[j * stride * 4 + k * 4 + b];
                sum += p;
            }
        }
    }
    return fabsf(sum) < 1e-5f ? 0.0f : sum;
}

/* dequantize_embedding_core with a block's four centroids (the get_row_core
 * call, compute/quantize/dequantize.rs:6-42): MSB-first codes, 00/01/11/10 ->
 * c0/c1/c2/c3. */
void orc_dequant_2bit(const uint8_t *packed, size_t n_bytes, const float *c, float *out) {
    for (size_t i = 0; i < n_bytes; i++)
        for (int j = 0; j < 4; j++) {
            const int bits = (packed[i] >> ((3 - j) * 2)) & 3;
            out[4 * i + j] = bits == 0 ? c[0] : bits == 1 ? c[1] : bits == 3 ? c[2] : c[3];
        }
}

/* dot_product, x86 AVX2+FMA branch — src/compute/kernels/dot.rs:43-67. */
float orc_dot_f32(const float *a, const float *b, size_t n) {
    __m256 acc = _mm256_setzero_ps();
    size_t i = 0;
    while (i + 8 <= n) {
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc);
        i += 8;
    }
    __m128 hi = _mm256_extractf128_ps(acc, 1);
    __m128 lo = _mm256_castps256_ps128(acc);
    __m128 sum128 = _mm_add_ps(lo, hi);
    __m128 shuf = _mm_movehdup_ps(sum128);
    __m128 sums = _mm_add_ps(sum128, shuf);
    __m128 shuf2 = _mm_movehl_ps(sums, sums);
    __m128 result = _mm_add_ss(sums, shuf2);
    float sum = _mm_cvtss_f32(result);
    while (i < n) {
        float p = a[i] * b[i];
        sum += p;
        i += 1;
    }
    return sum;
}

/* rms_norm, x86 AVX2+FMA branch — src/compute/kernels/norm.rs:52-88. */
void orc_rms_norm(const float *x, const float *weight, float eps, size_t n, float *out) {
    __m256 acc = _mm256_setzero_ps();
    size_t i = 0;
    while (i + 8 <= n) {
        __m256 vx = _mm256_loadu_ps(x + i);
        acc = _mm256_fmadd_ps(vx, vx, acc);
        i += 8;
    }
    __m128 hi = _mm256_extractf128_ps(acc, 1);
    __m128 lo = _mm256_castps256_ps128(acc);
    __m128 sum128 = _mm_add_ps(lo, hi);
    __m128 shuf = _mm_movehdup_ps(sum128);
    __m128 sums = _mm_add_ps(sum128, shuf);
    __m128 shuf2 = _mm_movehl_ps(sums, sums);
    __m128 result = _mm_add_ss(sums, shuf2);
    float sum_sq = _mm_cvtss_f32(result);
    while (i < n) {
        float p = x[i] * x[i];
        sum_sq += p;
        i += 1;
    }
    float mean = sum_sq / (float)n;
    float inv_rms = 1.0f / sqrtf(mean + eps);
    __m256 inv_v = _mm256_set1_ps(inv_rms);
    i = 0;
    while (i + 8 <= n) {
        __m256 vx = _mm256_loadu_ps(x + i);
        __m256 vw = _mm256_loadu_ps(weight + i);
        _mm256_storeu_ps(out + i, _mm256_mul_ps(_mm256_mul_ps(vx, inv_v), vw));
        i += 8;
    }
    while (i < n) {
        float t = x[i] * inv_rms;
        out[i] = t * weight[i];
        i += 1;
    }
}

/* swiglu_balanced — src/compute/kernels/activation.rs:35-51.  Sigmoid of the
 * clamped gate, product with the raw gate; h_scale is unused upstream. */
void orc_swiglu_balanced(const float *gate, const float *up, float *out, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) {
        float g = gate[i], u = up[i];
        float gs = g;
        if (gs < -64.0f) gs = -64.0f;
        if (gs > 64.0f) gs = 64.0f;
        float sig;
        if (gs >= 0.0f) {
            sig = 1.0f / (1.0f + ORC_EXPF(-gs));
        } else {
            float ex = ORC_EXPF(gs);
            sig = ex / (1.0f + ex);
        }
        float silu = g * sig;
        out[i] = silu * u;
    }
}

static int cmp_desc(const void *pa, const void *pb) {
    float a = *(const float *)pa, b = *(const float *)pb;
    if (a > b) return -1;
    if (a < b) return 1;
    return 0;
}

/* lateral_inhibition_kwta — src/compute/kernels/lut.rs:45-61.  threshold is
 * the k-th largest; strictly smaller values become -1e9; ties survive. */
void orc_kwta(float *scores, size_t n, size_t k) {
    if (n <= k || k == 0) return;
    float *sorted = (float *)malloc(n * sizeof(float));
    memcpy(sorted, scores, n * sizeof(float));
    qsort(sorted, n, sizeof(float), cmp_desc);
    float thr = sorted[k - 1];
    free(sorted);
    for (size_t i = 0; i < n; i++)
        if (scores[i] < thr) scores[i] = -1e9f;
}

/* Rotary embedding closure of forward_attention_core —
 * src/nn/attention.rs:62-82 (split pairs (i, i+hd/2); else (2i, 2i+1)). */
void orc_rope(float *vec, int heads, int head_dim, float rope_base, size_t pos, int is_split) {
    for (int h = 0; h < heads; h++) {
        int hs = h * head_dim;
        for (int i = 0; i < head_dim / 2; i++) {
            float expo = (2.0f * (float)i) / (float)head_dim;
            float freq = 1.0f / powf(rope_base, expo);
            float theta = (float)pos * freq;
            float s = sinf(theta), c = cosf(theta);
            int a, b;
            if (is_split) { a = hs + i; b = hs + i + head_dim / 2; }
            else { a = hs + 2 * i; b = hs + 2 * i + 1; }
            float v0 = vec[a], v1 = vec[b];
            float t0 = v0 * c, t1 = v1 * s, t2 = v0 * s, t3 = v1 * c;
            vec[a] = t0 - t1;
            vec[b] = t2 + t3;
        }
    }
}

/* GQA softmax attention over the (already appended) cache —
 * src/nn/attention.rs:87-127.  k_cache/v_cache are [seq_len][n_head_kv*hd]. */
void orc_attention(const float *q_rope, const float *k_cache, const float *v_cache,
                   size_t seq_len, int n_head, int n_head_kv, int head_dim, float *out) {
    int n_groups = n_head / n_head_kv;
    float scale = 1.0f / sqrtf((float)head_dim);
    size_t kv_stride = (size_t)n_head_kv * head_dim;
#pragma omp parallel for schedule(static)
    for (int h = 0; h < n_head; h++) {
        int kv_h = h / n_groups;
        size_t off = (size_t)kv_h * head_dim;
        const float *q = q_rope + (size_t)h * head_dim;
        float *scores = (float *)malloc((seq_len ? seq_len : 1) * sizeof(float));
        float max_s = -INFINITY;
        for (size_t t = 0; t < seq_len; t++) {
            float s = orc_dot_f32(q, k_cache + t * kv_stride + off, head_dim) * scale;
            scores[t] = s;
            if (s > max_s) max_s = s;
        }
        float sum_e = 0.0f;
        for (size_t t = 0; t < seq_len; t++) {
            scores[t] = ORC_EXPF(scores[t] - max_s);
            sum_e += scores[t];
        }
        float inv_s = 1.0f / (sum_e + 1e-12f);
        float *ho = out + (size_t)h * head_dim;
        for (int i = 0; i < head_dim; i++) ho[i] = 0.0f;
        for (size_t t = 0; t < seq_len; t++) {
            float w = scores[t] * inv_s;
            const float *vh = v_cache + t * kv_stride + off;
            for (int i = 0; i < head_dim; i++) {
                float p = w * vh[i];
                ho[i] += p;
            }
        }
        free(scores);
    }
}

/* A GenomicLinear as the oracle sees it (src/nn/linear/mod.rs:36-57). */
typedef struct {
    int kind;              /* 0 = GenomicF32, 1 = GenomicQ4_0, 2 = Genomic4Bit (LUT), 3 = GenomicQ8_0,
                              4 = Genomic2Bit */
    int64_t out_features;
    int64_t in_features;
    const uint8_t *db;     /* weight bytes as stored in the .flat blob */
    int64_t db_len;
    const float *centroids; /* expanded LUT / centroids (init.rs:109-139), kinds 2 and 4 */
    int64_t centroids_len;
    const float *bias;
    int64_t bias_len;
    /* sparse f16 anchors (init.rs:61-107); n_anchors == 0 when absent */
    const uint32_t *anchor_indices;
    const uint16_t *anchor_values;
    const int64_t *anchor_row_ptrs; /* out_features + 1 entries */
    int64_t n_anchors;
} orc_linear;

/* GenomicLinear::compute_single_row — src/nn/linear/forward.rs:11-117
 * (block_size 32; the modulation factors are 1: load_genomic sets no topology,
 * flat_reader.rs:235). */
static float compute_single_row(const orc_linear *L, int64_t i, const float *input, int64_t in_len) {
    const int64_t block_size = 32;
    int64_t n_blocks = L->in_features / block_size;
    float sum = 0.0f;
    if (L->kind == 0) {
        int64_t row_off = i * L->in_features;
        const float *row = (const float *)L->db + row_off;
        if (L->in_features == in_len) {
            sum = orc_dot_f32(input, row, (size_t)in_len);
        } else {
            int64_t n = L->in_features < in_len ? L->in_features : in_len;
            float s = 0.0f;
            for (int64_t t = 0; t < n; t++) { float p = input[t] * row[t]; s += p; }
            sum = s;
        }
    } else if (L->kind == 1) {
        int64_t row_off = i * n_blocks;
        int64_t total_blocks = L->db_len / Q4_0_BLOCK_BYTES;
        if (n_blocks > 0 && row_off + n_blocks <= total_blocks)
            sum = orc_dot_q4_0_avx2(L->db + row_off * Q4_0_BLOCK_BYTES, input, (size_t)n_blocks);
    } else if (L->kind == 3) {
        int64_t row_off = i * n_blocks;
        int64_t total_blocks = L->db_len / Q8_0_BLOCK_BYTES;
        if (n_blocks > 0 && row_off + n_blocks <= total_blocks)
            sum = orc_dot_q8_0_avx2(L->db + row_off * Q8_0_BLOCK_BYTES, input, (size_t)n_blocks);
    } else if (L->kind == 2) {
        const int64_t stride = block_size / 2;
        int64_t row_off = i * n_blocks * stride;
        int64_t c_start = i * n_blocks * 16;
        const float *c = NULL;
        if (L->centroids_len >= c_start + n_blocks * 16) c = L->centroids + c_start;
        else if (L->centroids_len >= 16) c = L->centroids;
        if (n_blocks > 0 && row_off + n_blocks * stride <= L->db_len && c)
            sum = orc_dot_4bit(L->db + row_off, input, c, (size_t)stride, (size_t)n_blocks);
    } else if (L->kind == 4) {
        /* forward.rs:33-57: the row's centroids, else the table's start (the
         * dot then reads 4 floats per block from there) */
        const int64_t stride = block_size / 4;
        int64_t row_off = i * n_blocks * stride;
        int64_t c_start = i * n_blocks * 4;
        const float *c = NULL;
        if (L->centroids_len >= c_start + n_blocks * 4) c = L->centroids + c_start;
        else if (L->centroids_len >= 4) c = L->centroids;
        if (n_blocks > 0 && row_off + n_blocks * stride <= L->db_len && c)
            sum = orc_dot_2bit(L->db + row_off, input, c, (size_t)stride, (size_t)n_blocks, NULL);
    }
    if (L->n_anchors > 0) {
        int64_t a_s = L->anchor_row_ptrs[i], a_e = L->anchor_row_ptrs[i + 1];
        if (a_s < a_e && a_e <= L->n_anchors) {
            for (int64_t k = a_s; k < a_e; k++) {
                int64_t col = (int64_t)L->anchor_indices[k] % L->in_features;
                if (col < in_len) {
                    float p = input[col] * h2f(L->anchor_values[k]);
                    sum += p;
                }
            }
        }
    }
    if (i < L->bias_len) sum += L->bias[i];
    return sum;
}

/* GenomicLinear::forward_core — src/nn/linear/forward.rs:119-132; the rayon
 * row loop becomes an OpenMP row loop (rows are independent). */
void orc_linear_forward(const orc_linear *L, const float *input, int64_t in_len, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < L->out_features; i++)
        out[i] = compute_single_row(L, i, input, in_len);
}

/* One row for a single-row check (compute_single_row). */
float orc_linear_row(const orc_linear *L, int64_t i, const float *input, int64_t in_len) {
    return compute_single_row(L, i, input, in_len);
}

/* GenomicLinear::get_row_core — src/nn/linear/forward.rs:195-285 for the
 * F32, Q4_0, Q8_0, LUT-4bit and 2-bit variants (embedding lookup). */
void orc_linear_get_row(const orc_linear *L, int64_t idx, float *res) {
    int64_t K = L->in_features;
    for (int64_t t = 0; t < K; t++) res[t] = 0.0f;
    if (L->out_features == 0 || K == 0) return;
    int64_t safe = idx % L->out_features;
    int64_t n_blocks = K / 32;
    if (L->kind == 0) {
        int64_t off = safe * K;
        if (off + K <= L->db_len / 4) memcpy(res, (const float *)L->db + off, (size_t)K * 4);
    } else if (L->kind == 1) {
        int64_t off = safe * n_blocks;
        if (off + n_blocks <= L->db_len / Q4_0_BLOCK_BYTES)
            orc_q4_0_dequant(L->db + off * Q4_0_BLOCK_BYTES, (size_t)n_blocks, res);
    } else if (L->kind == 3) {
        int64_t off = safe * n_blocks;
        if (off + n_blocks <= L->db_len / Q8_0_BLOCK_BYTES)
            orc_q8_0_dequant(L->db + off * Q8_0_BLOCK_BYTES, (size_t)n_blocks, res);
    } else if (L->kind == 2) {
        int64_t off = safe * n_blocks * 16;
        if (off + n_blocks * 16 <= L->db_len) {
            for (int64_t b = 0; b < n_blocks; b++) {
                int64_t c_off = (safe * n_blocks + b) * 16;
                const float *c;
                static const float zeros[16] = {0};
                if (L->centroids_len == 16) c = L->centroids;
                else if (c_off + 16 <= L->centroids_len) c = L->centroids + c_off;
                else if (L->centroids_len > 0) c = L->centroids;
                else c = zeros;
                for (int k = 0; k < 16; k++) {
                    uint8_t byte = L->db[off + b * 16 + k];
                    res[b * 32 + k * 2] = c[byte >> 4];
                    res[b * 32 + k * 2 + 1] = c[byte & 0x0F];
                }
            }
        }
    } else if (L->kind == 4) {
        /* forward.rs:210-237: per block the row's own centroids if present,
         * else the first four (a table of fewer than 4 floats is refused by
         * the loader: the reference would index past it) */
        int64_t off = safe * n_blocks * 8;
        if (off + n_blocks * 8 <= L->db_len) {
            static const float zeros[4] = {0};
            for (int64_t b = 0; b < n_blocks; b++) {
                int64_t c_off = (safe * n_blocks + b) * 4;
                const float *c;
                if (L->centroids_len == 4) c = L->centroids;
                else if (c_off + 4 <= L->centroids_len) c = L->centroids + c_off;
                else if (L->centroids_len > 0) c = L->centroids;
                else c = zeros;
                orc_dequant_2bit(L->db + off + b * 8, 8, c, res + b * 32);
            }
        }
    }
}
