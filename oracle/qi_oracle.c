/*
 * qi_oracle.c -- CPU restatement of the reference's QIPACK INT4 linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP product is
 * compared against, and the CPU baseline that bench.py times beside it.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load the
 * library built from it; the product never links, loads or calls it.
 *
 * Every function cites the reference file:line whose arithmetic it restates
 * (paths relative to the reference tree netdur/qwen-image-cplus 0.2.5).  The
 * operation order follows the reference statement literally, because several
 * outputs (activation codes, weight codes, fp16 scales) must be bit-exact.
 *
 * Compiled with -ffp-contract=off so that a*b+c is two roundings unless the
 * reference contracts it (then fmaf() is written out explicitly).
 *
 * Pinning (what checks each function, beyond restating it):
 *   half_*           KATs half.cplus:81-90; exhaustive f16->f32->f16 round
 *                    trip; IEEE RNE ties checked against numpy float16.
 *   hadamard256      involution KAT int4_pack.cplus:854-869; equality with
 *                    the dense 4x4 Kronecker matrix (brute force); norm.
 *   quantize_*_group KATs int4_pack.cplus:871-938; brute-force search over
 *                    all 7 clip candidates recomputed independently in tests.
 *   quantize_acts    closed form gemm.cu:41-51: zero group, spike, RNE ties.
 *   w4a4_gemm        exact int32 group partials by brute force; float64
 *                    formula bench_w4a4.cu:383-394 as the tolerance anchor.
 *   w4a16_gemm       float64 matmul of the dequantised fp16 weights.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QO_EXPORT __attribute__((visibility("default")))

/* ---------------------------------------------------------------- fp16 -- */

static inline float f32_from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* half.cplus:12-34 (to_f32): exact widening, subnormals normalised. */
QO_EXPORT float qo_half_to_f32(uint16_t bits) {
    uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
    uint32_t exponent = ((uint32_t)bits >> 10) & 0x1Fu;
    uint32_t mantissa = (uint32_t)bits & 0x03FFu;
    if (exponent == 0) {
        if (mantissa == 0) return f32_from_bits(sign);
        int32_t unbiased = -14;
        while ((mantissa & 0x0400u) == 0) { mantissa <<= 1; unbiased -= 1; }
        mantissa &= 0x03FFu;
        return f32_from_bits(sign | ((uint32_t)(unbiased + 127) << 23) | (mantissa << 13));
    }
    if (exponent == 31) return f32_from_bits(sign | 0x7F800000u | (mantissa << 13));
    return f32_from_bits(sign | ((exponent + 127 - 15) << 23) | (mantissa << 13));
}

/* half.cplus:36-75 (from_f32): round to nearest even, subnormal results,
 * overflow to infinity, NaN -> 0x7E00. */
QO_EXPORT uint16_t qo_half_from_f32(float value) {
    uint32_t bits = f32_bits(value);
    uint32_t sign = (bits >> 16) & 0x8000u;
    uint32_t exponent = (bits >> 23) & 0xFFu;
    uint32_t mantissa = bits & 0x7FFFFFu;
    if (exponent == 0xFF) return (uint16_t)(mantissa == 0 ? (sign | 0x7C00u) : (sign | 0x7E00u));
    int32_t half_exponent = (int32_t)exponent - 127 + 15;
    if (half_exponent >= 31) return (uint16_t)(sign | 0x7C00u);
    if (half_exponent <= 0) {
        if (half_exponent < -10) return (uint16_t)sign;
        uint32_t significand = mantissa | 0x800000u;
        uint32_t shift = (uint32_t)(14 - half_exponent);
        uint32_t rounded = significand >> shift;
        uint32_t mask = (1u << shift) - 1u;
        uint32_t remainder = significand & mask;
        uint32_t halfway = 1u << (shift - 1u);
        if (remainder > halfway || (remainder == halfway && (rounded & 1u))) rounded += 1u;
        return (uint16_t)(sign | rounded);
    }
    uint32_t encoded = sign | ((uint32_t)half_exponent << 10) | (mantissa >> 13);
    uint32_t remainder = mantissa & 0x1FFFu;
    if (remainder > 0x1000u || (remainder == 0x1000u && (encoded & 1u))) encoded += 1u;
    return (uint16_t)encoded;
}

/* half.cplus:77-79 (round_f32). */
QO_EXPORT float qo_half_round(float value) { return qo_half_to_f32(qo_half_from_f32(value)); }

QO_EXPORT void qo_f32_to_f16(const float *source, uint16_t *out, uint64_t count) {
    /* ops.cu:204-212 (f32_to_f16_kernel): __float2half is RNE, same as above. */
    for (uint64_t i = 0; i < count; ++i) out[i] = qo_half_from_f32(source[i]);
}

/* ---------------------------------------------------------------- H256 -- */

/* int4_pack.cplus:249-273 (hadamard_256_in_place) and gemm.cu:28-39: radix-4
 * butterfly, strides 1, 4, 16, 64; exact fp32 operation order. */
QO_EXPORT void qo_hadamard256(float *values) {
    for (int stride = 1; stride < 256; stride *= 4) {
        int span = stride * 4;
        for (int base = 0; base < 256; base += span) {
            for (int offset = 0; offset < stride; ++offset) {
                float a = values[base + offset];
                float b = values[base + stride + offset];
                float c = values[base + 2 * stride + offset];
                float d = values[base + 3 * stride + offset];
                values[base + offset] = (a + b + c - d) * 0.5f;
                values[base + stride + offset] = (a + b - c + d) * 0.5f;
                values[base + 2 * stride + offset] = (a - b + c + d) * 0.5f;
                values[base + 3 * stride + offset] = (-a + b + c + d) * 0.5f;
            }
        }
    }
}

/* ---------------------------------------------------------- quantizers -- */

/* int4_pack.cplus:237-245 (clip_candidate). */
static double clip_candidate(int index) {
    static const double table[7] = {1.0, 0.95, 0.9, 0.85, 0.8, 0.75, 0.7};
    return table[index < 7 ? index : 6];
}

static const float SCALE_FLOOR = 0.000000059604645f; /* int4_pack.cplus:53 */

static inline float fmin_ref(float a, float b) { return b < a ? b : a; }
static inline float fmax_ref(float a, float b) { return b > a ? b : a; }

/* int4_pack.cplus:275-320 (quantize_affine_group), scheme 5.  Unsigned codes
 * 0..15, fp16 scale and fp16 minimum; first strictly smaller error wins; the
 * squared error is summed sequentially in fp32. */
QO_EXPORT void qo_quantize_affine_group(const float *values, int group, int clip, uint8_t *codes,
                                        uint16_t *scale_bits, uint16_t *minimum_bits) {
    float low = values[0], high = values[0];
    for (int i = 1; i < group; ++i) { low = fmin_ref(low, values[i]); high = fmax_ref(high, values[i]); }
    float best_error = 0.0f;
    int candidates = clip ? 7 : 1;
    for (int candidate = 0; candidate < candidates; ++candidate) {
        float center = (high + low) * 0.5f;
        float half_range = (high - low) * (float)(0.5 * clip_candidate(candidate));
        float minimum = qo_half_round(center - half_range);
        float scale = qo_half_round(fmax_ref((center + half_range - minimum) / 15.0f, SCALE_FLOOR));
        float error = 0.0f;
        for (int i = 0; i < group; ++i) {
            float code = fmin_ref(fmax_ref(rintf((values[i] - minimum) / scale), 0.0f), 15.0f);
            float difference = code * scale + minimum - values[i];
            error = error + difference * difference;
        }
        if (candidate == 0 || error < best_error) {
            best_error = error;
            *scale_bits = qo_half_from_f32(scale);
            *minimum_bits = qo_half_from_f32(minimum);
            for (int i = 0; i < group; ++i)
                codes[i] = (uint8_t)fmin_ref(fmax_ref(rintf((values[i] - minimum) / scale), 0.0f), 15.0f);
        }
    }
}

/* int4_pack.cplus:322-363 (quantize_symmetric_group), scheme 6.  Signed codes
 * -7..7 stored as two's-complement nibbles, scale = fp16(peak * f32(c / 7)). */
QO_EXPORT void qo_quantize_symmetric_group(const float *values, int group, int clip, uint8_t *codes,
                                           uint16_t *scale_bits) {
    float peak = 0.0f;
    for (int i = 0; i < group; ++i) peak = fmax_ref(peak, fabsf(values[i]));
    float best_error = 0.0f;
    int candidates = clip ? 7 : 1;
    for (int candidate = 0; candidate < candidates; ++candidate) {
        float factor = (float)(clip_candidate(candidate) / 7.0);
        float scale = qo_half_round(fmax_ref(peak * factor, SCALE_FLOOR));
        float error = 0.0f;
        for (int i = 0; i < group; ++i) {
            float code = fmin_ref(fmax_ref(rintf(values[i] / scale), -7.0f), 7.0f);
            float difference = code * scale - values[i];
            error = error + difference * difference;
        }
        if (candidate == 0 || error < best_error) {
            best_error = error;
            *scale_bits = qo_half_from_f32(scale);
            for (int i = 0; i < group; ++i) {
                float code = fmin_ref(fmax_ref(rintf(values[i] / scale), -7.0f), 7.0f);
                codes[i] = (uint8_t)(((int32_t)code) & 15);
            }
        }
    }
}

/* int4_pack.cplus:381-425 (quantize_rows) over rows [start, end): fp16 row ->
 * f32, H256 per 256-chunk when rotating (W4A4), per-group quantiser, nibble
 * packing with the even input column in the low nibble (:414-418). */
static void quantize_rows(const uint16_t *source, int64_t inputs, int group, int rotate, int clip,
                          uint8_t *codes, uint16_t *scales, uint16_t *minimums, int64_t start, int64_t end) {
    float *row = (float *)malloc((size_t)inputs * sizeof(float));
    uint8_t group_codes[256];
    int64_t groups = inputs / group;
    for (int64_t r = start; r < end; ++r) {
        for (int64_t c = 0; c < inputs; ++c) row[c] = qo_half_to_f32(source[r * inputs + c]);
        if (rotate)
            for (int64_t chunk = 0; chunk < inputs; chunk += 256) qo_hadamard256(row + chunk);
        for (int64_t g = 0; g < groups; ++g) {
            int64_t s = g * group;
            uint16_t scale_bits = 0, minimum_bits = 0;
            if (rotate) {
                qo_quantize_symmetric_group(row + s, group, clip, group_codes, &scale_bits);
            } else {
                qo_quantize_affine_group(row + s, group, clip, group_codes, &scale_bits, &minimum_bits);
                minimums[r * groups + g] = minimum_bits;
            }
            scales[r * groups + g] = scale_bits;
            for (int p = 0; p < group; p += 2)
                codes[(r * inputs + s + p) / 2] = (uint8_t)(group_codes[p] | (group_codes[p + 1] << 4));
        }
    }
    free(row);
}

/* int4_pack.cplus:427-468 (quantize_matrix).  scheme 5 = W4A16 affine,
 * scheme 6 = W4A4 H256 symmetric.  Rows are independent, so the threaded
 * split does not change any output. */
QO_EXPORT int qo_quantize_matrix(const uint16_t *source, int64_t outputs, int64_t inputs, int scheme, int group,
                                 int clip, uint8_t *codes, uint16_t *scales, uint16_t *minimums) {
    if (group < 32 || group > 256 || group % 2 || 256 % group) return 2; /* int4_pack.cplus:520-525 */
    int rotate = scheme == 6;
    /* The rotation needs whole 256-chunks.  The reference writer demands
     * inputs % 256 of every block matrix (int4_pack.cplus:590-593); that is a
     * container rule, checked by the pack writer, not by this arithmetic. */
    if (rotate && inputs % 256) return 1;
    if (inputs % group) return 1;
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t r = 0; r < outputs; ++r)
        quantize_rows(source, inputs, group, rotate, clip, codes, scales, minimums, r, r + 1);
    return 0;
}

/* gemm.cu:22-52 (quantize_activations_kernel) for one f32 row already loaded:
 * H256 per 256-chunk, then per 64-group scale = fp16(max(peak / 7, 2^-24)),
 * codes = clamp(rint(v / scale), -7, 7), packed (c0 & 15) | (c1 & 15) << 4.
 * No activation clipping. */
static void quantize_activation_row(float *row, int k, uint8_t *codes, uint16_t *scales) {
    for (int chunk = 0; chunk < k; chunk += 256) qo_hadamard256(row + chunk);
    for (int g = 0; g < k / 64; ++g) {
        float peak = 0.0f;
        for (int i = 0; i < 64; ++i) peak = fmaxf(peak, fabsf(row[g * 64 + i]));
        uint16_t scale_half = qo_half_from_f32(fmaxf(peak / 7.0f, 5.9604645e-08f));
        float scale = qo_half_to_f32(scale_half);
        for (int lane = 0; lane < 32; ++lane) {
            int c0 = (int)fminf(fmaxf(rintf(row[g * 64 + 2 * lane] / scale), -7.0f), 7.0f);
            int c1 = (int)fminf(fmaxf(rintf(row[g * 64 + 2 * lane + 1] / scale), -7.0f), 7.0f);
            codes[g * 32 + lane] = (uint8_t)((c0 & 0xF) | ((c1 & 0xF) << 4));
        }
        scales[g] = scale_half;
    }
}

/* gemm.cu:54-57 (qi_w4a4_quantize_activations), fp32 input. */
QO_EXPORT void qo_quantize_activations_f32(const float *x, uint8_t *codes, uint16_t *scales, int64_t m, int k) {
#pragma omp parallel
    {
        float *row = (float *)malloc((size_t)k * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < m; ++r) {
            memcpy(row, x + r * k, (size_t)k * sizeof(float));
            quantize_activation_row(row, k, codes + r * (k / 2), scales + r * (k / 64));
        }
        free(row);
    }
}

/* bench_w4a4.cu:30-66 (fp16-input twin): the row is widened exactly, then the
 * same arithmetic as the fp32 entry point. */
QO_EXPORT void qo_quantize_activations_f16(const uint16_t *x, uint8_t *codes, uint16_t *scales, int64_t m, int k) {
#pragma omp parallel
    {
        float *row = (float *)malloc((size_t)k * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < m; ++r) {
            for (int i = 0; i < k; ++i) row[i] = qo_half_to_f32(x[r * k + i]);
            quantize_activation_row(row, k, codes + r * (k / 2), scales + r * (k / 64));
        }
        free(row);
    }
}

/* Rotated fp32 row only (H256 of gemm.cu:28-39), exposed so tests can feed the
 * identical rotated input to both quantisers. */
QO_EXPORT void qo_rotate_rows(float *x, int64_t m, int k) {
    for (int64_t r = 0; r < m; ++r)
        for (int chunk = 0; chunk < k; chunk += 256) qo_hadamard256(x + r * k + chunk);
}

/* ---------------------------------------------------------------- GEMMs -- */

/* bench_w4a4.cu:376-380 (nibble): signed two's-complement nibble k of a row. */
static inline int nibble_signed(const uint8_t *row_codes, int64_t col) {
    uint8_t byte = row_codes[col / 2];
    int v = (col % 2 == 0) ? (byte & 0xF) : (byte >> 4);
    return v >= 8 ? v - 16 : v;
}

/* Exact int32 per-group partial sums P[m, n, g] = sum_{k in g} qa * qw
 * (gemm.cu:139-158).  Output layout [m][n][g]. */
QO_EXPORT void qo_w4a4_partials(const uint8_t *a_codes, const uint8_t *w_codes, int32_t *partials,
                                int64_t m, int64_t n, int64_t k) {
    int64_t groups = k / 64;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t r = 0; r < m; ++r)
        for (int64_t c = 0; c < n; ++c)
            for (int64_t g = 0; g < groups; ++g) {
                int32_t sum = 0;
                for (int64_t i = g * 64; i < (g + 1) * 64; ++i)
                    sum += nibble_signed(a_codes + r * (k / 2), i) * nibble_signed(w_codes + c * (k / 2), i);
                partials[(r * n + c) * groups + g] = sum;
            }
}

/* gemm.cu:159-168: y = sum over ascending groups of fmaf((float)P, sa * sw, y)
 * (nvcc contracts the accumulate into an fma; sa * sw is formed first). */
QO_EXPORT void qo_w4a4_gemm(const uint8_t *a_codes, const uint16_t *a_scales, const uint8_t *w_codes,
                            const uint16_t *w_scales, float *y, int64_t m, int64_t n, int64_t k) {
    int64_t groups = k / 64;
#pragma omp parallel
    {
        int8_t *arow = (int8_t *)malloc((size_t)k);
#pragma omp for schedule(dynamic, 1)
        for (int64_t r = 0; r < m; ++r) {
            for (int64_t i = 0; i < k; ++i) arow[i] = (int8_t)nibble_signed(a_codes + r * (k / 2), i);
            for (int64_t c = 0; c < n; ++c) {
                const uint8_t *wc = w_codes + c * (k / 2);
                float acc = 0.0f;
                for (int64_t g = 0; g < groups; ++g) {
                    int32_t sum = 0;
                    for (int64_t i = g * 64; i < (g + 1) * 64; i += 2) {
                        uint8_t byte = wc[i / 2];
                        int lo = byte & 0xF, hi = byte >> 4;
                        sum += arow[i] * (lo >= 8 ? lo - 16 : lo) + arow[i + 1] * (hi >= 8 ? hi - 16 : hi);
                    }
                    float sa = qo_half_to_f32(a_scales[r * groups + g]);
                    float sw = qo_half_to_f32(w_scales[c * groups + g]);
                    acc = fmaf((float)sum, sa * sw, acc);
                }
                y[r * n + c] = acc;
            }
        }
        free(arow);
    }
}

/* bench_w4a4.cu:383-394 (reference_gemm): the same formula in float64. */
QO_EXPORT void qo_w4a4_gemm_f64(const uint8_t *a_codes, const uint16_t *a_scales, const uint8_t *w_codes,
                                const uint16_t *w_scales, double *y, int64_t m, int64_t n, int64_t k) {
    int64_t groups = k / 64;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t r = 0; r < m; ++r)
        for (int64_t c = 0; c < n; ++c) {
            double total = 0.0;
            for (int64_t g = 0; g < groups; ++g) {
                int32_t sum = 0;
                for (int64_t i = g * 64; i < (g + 1) * 64; ++i)
                    sum += nibble_signed(a_codes + r * (k / 2), i) * nibble_signed(w_codes + c * (k / 2), i);
                total += (double)sum * (double)qo_half_to_f32(a_scales[r * groups + g]) *
                         (double)qo_half_to_f32(w_scales[c * groups + g]);
            }
            y[r * n + c] = total;
        }
}

/* gemm.cu:222-230 and bench_w4a16.cu:117-126: w = fp16(fmaf(code, scale,
 * minimum)), unsigned codes, even column in the low nibble.  Output [n, k]. */
QO_EXPORT void qo_w4a16_dequantize(const uint8_t *codes, const uint16_t *scales, const uint16_t *minimums,
                                   uint16_t *weights, int64_t n, int64_t k) {
    int64_t groups = k / 64;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r)
        for (int64_t i = 0; i < k; ++i) {
            uint8_t byte = codes[r * (k / 2) + i / 2];
            float code = (float)((i % 2 == 0) ? (byte & 0x0F) : (byte >> 4));
            float scale = qo_half_to_f32(scales[r * groups + i / 64]);
            float minimum = qo_half_to_f32(minimums[r * groups + i / 64]);
            weights[r * k + i] = qo_half_from_f32(fmaf(code, scale, minimum));
        }
}

QO_EXPORT void qo_sgemm_nt(const float *x, const float *w, float *y, int64_t m, int64_t n, int64_t k);

/* y[m, n] = sum_k x[m, k] * w[n, k] over fp16 operands.  gemm.cu:238-252
 * accumulates exact fp16 products in fp32 inside the matrix unit; the oracle
 * accumulates in float64 (precise = 1), the tolerance anchor, or in fp32
 * with a blocked loop (precise = 0), the CPU baseline kernel. */
QO_EXPORT void qo_gemm_f16(const uint16_t *x, const uint16_t *w, float *y, int64_t m, int64_t n, int64_t k,
                           int precise) {
    if (precise) {
        float *wf = (float *)malloc((size_t)(n * k) * sizeof(float));
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n * k; ++i) wf[i] = qo_half_to_f32(w[i]);
#pragma omp parallel
        {
            double *xr = (double *)malloc((size_t)k * sizeof(double));
#pragma omp for schedule(dynamic, 1)
            for (int64_t r = 0; r < m; ++r) {
                for (int64_t i = 0; i < k; ++i) xr[i] = qo_half_to_f32(x[r * k + i]);
                for (int64_t c = 0; c < n; ++c) {
                    const float *wr = wf + c * k;
                    double total = 0.0;
                    for (int64_t i = 0; i < k; ++i) total += xr[i] * (double)wr[i];
                    y[r * n + c] = (float)total;
                }
            }
            free(xr);
        }
        free(wf);
        return;
    }
    /* Blocked fp32: widen once, then 4 x 4 register tiles over k. */
    float *xf = (float *)malloc((size_t)(m * k) * sizeof(float));
    float *wf = (float *)malloc((size_t)(n * k) * sizeof(float));
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m * k; ++i) xf[i] = qo_half_to_f32(x[i]);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n * k; ++i) wf[i] = qo_half_to_f32(w[i]);
    qo_sgemm_nt(xf, wf, y, m, n, k);
    free(xf);
    free(wf);
}

/* Blocked fp32 y = x . w^T used by the CPU baseline (no reference
 * counterpart: the reference has no CPU GEMM for this path). */
QO_EXPORT void qo_sgemm_nt(const float *x, const float *w, float *y, int64_t m, int64_t n, int64_t k) {
    const int64_t TB = 64;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int64_t r0 = 0; r0 < m; r0 += TB)
        for (int64_t c0 = 0; c0 < n; c0 += TB) {
            int64_t r1 = r0 + TB < m ? r0 + TB : m, c1 = c0 + TB < n ? c0 + TB : n;
            for (int64_t r = r0; r < r1; r += 4)
                for (int64_t c = c0; c < c1; c += 4) {
                    float acc[4][4] = {{0}};
                    int rr = (int)(r1 - r < 4 ? r1 - r : 4), cc = (int)(c1 - c < 4 ? c1 - c : 4);
                    if (rr == 4 && cc == 4) {
                        const float *x0 = x + r * k, *x1 = x0 + k, *x2 = x1 + k, *x3 = x2 + k;
                        const float *w0 = w + c * k, *w1 = w0 + k, *w2 = w1 + k, *w3 = w2 + k;
                        for (int64_t i = 0; i < k; ++i) {
                            float a0 = x0[i], a1 = x1[i], a2 = x2[i], a3 = x3[i];
                            float b0 = w0[i], b1 = w1[i], b2 = w2[i], b3 = w3[i];
                            acc[0][0] += a0 * b0; acc[0][1] += a0 * b1; acc[0][2] += a0 * b2; acc[0][3] += a0 * b3;
                            acc[1][0] += a1 * b0; acc[1][1] += a1 * b1; acc[1][2] += a1 * b2; acc[1][3] += a1 * b3;
                            acc[2][0] += a2 * b0; acc[2][1] += a2 * b1; acc[2][2] += a2 * b2; acc[2][3] += a2 * b3;
                            acc[3][0] += a3 * b0; acc[3][1] += a3 * b1; acc[3][2] += a3 * b2; acc[3][3] += a3 * b3;
                        }
                    } else {
                        for (int a = 0; a < rr; ++a)
                            for (int b = 0; b < cc; ++b)
                                for (int64_t i = 0; i < k; ++i) acc[a][b] += x[(r + a) * k + i] * w[(c + b) * k + i];
                    }
                    for (int a = 0; a < rr; ++a)
                        for (int b = 0; b < cc; ++b) y[(r + a) * n + c + b] = acc[a][b];
                }
        }
}

/* W4A16 for a few rows (the GEMV shapes) without materialising the
 * dequantised matrix: per weight row, fp16(fmaf(code, scale, minimum))
 * (gemm.cu:229-230) widened to fp32 -- formed once per group for the 16
 * possible codes -- then an fp32 dot product with each of the m fp16 input
 * rows.  The CPU baseline of the modulation linears (no
 * reference counterpart: the reference has no CPU GEMM for this path). */
QO_EXPORT void qo_w4a16_gemv(const uint16_t *x, const uint8_t *codes, const uint16_t *scales,
                             const uint16_t *minimums, float *y, int64_t m, int64_t n, int64_t k) {
    int64_t groups = k / 64;
    float *xf = (float *)malloc((size_t)(m * k) * sizeof(float));
    for (int64_t i = 0; i < m * k; ++i) xf[i] = qo_half_to_f32(x[i]);
#pragma omp parallel
    {
        float *wr = (float *)malloc((size_t)k * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < n; ++r) {
            for (int64_t g = 0; g < groups; ++g) {
                /* The group's 16 possible weights, then a table lookup per code. */
                float scale = qo_half_to_f32(scales[r * groups + g]);
                float minimum = qo_half_to_f32(minimums[r * groups + g]);
                float table[16];
                for (int c = 0; c < 16; ++c) table[c] = qo_half_round(fmaf((float)c, scale, minimum));
                const uint8_t *cb = codes + r * (k / 2) + g * 32;
                for (int i = 0; i < 32; ++i) {
                    wr[g * 64 + 2 * i] = table[cb[i] & 0x0F];
                    wr[g * 64 + 2 * i + 1] = table[cb[i] >> 4];
                }
            }
            for (int64_t a = 0; a < m; ++a) {
                float total = 0.0f;
                for (int64_t i = 0; i < k; ++i) total += xf[a * k + i] * wr[i];
                y[a * n + r] = total;
            }
        }
        free(wr);
    }
    free(xf);
}

/* ops.cu:156-160 (gelu_tanh_kernel). */
QO_EXPORT float qo_gelu_tanh(float v) {
    return 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
}

/* ------------------------------------------------------------- QIPACK1 -- */

/* int4_pack.cplus:47-48,151-159 (hash_update): FNV-1a 64. */
QO_EXPORT uint64_t qo_fnv1a(uint64_t hash, const uint8_t *bytes, uint64_t count) {
    for (uint64_t i = 0; i < count; ++i) hash = (hash ^ bytes[i]) * 1099511628211ull;
    return hash;
}

QO_EXPORT int qo_num_threads(void) {
#ifdef _OPENMP
    extern int omp_get_max_threads(void);
    return omp_get_max_threads();
#else
    return 1;
#endif
}
