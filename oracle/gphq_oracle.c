/*
 * gphq_oracle.c — CPU restatement of gophonic's quantized matrix-product
 * arithmetic. TEST INFRASTRUCTURE ONLY: the parity tests, the smoke check
 * and bench.py's cpu_baseline leg load this library as the checker and as the
 * CPU baseline. Nothing in the product (libgphq) links or calls it.
 *
 * Every function restates one reference function (file:line under the
 * gophonic tree) in plain C. Build with -O2 -ffp-contract=off: amd64 Go
 * (GOAMD64=v1) never fuses a multiply and an add, so neither may we.
 *
 * Pinning (how each function is checked independently of this file) is listed
 * in the header comment of each group; the checks themselves live in
 * tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OUTPUT_PANEL 64 /* q8gemm/packed.go:17 */
#define ACTIVATION_ROWS 16 /* q8gemm/packed.go:19 */

static inline uint32_t f32bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bitsf32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------ */
/* FP16 / BF16 conversions.
 * Pinned by: exhaustive 2^16 round trip, and bit-for-bit agreement with
 * numpy's IEEE float32->float16 (round to nearest even) over every finite
 * float16 neighbourhood and 10^6 random floats (tests/test_oracle.py). */

/* q8gemm/gemm.go:297-327 f32ToF16: nearest, ties to even; NaN -> sign|0x7e00;
 * exponent >= 31 -> signed infinity; exponent < -10 -> signed zero. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t b = f32bits(f);
    uint16_t sign = (uint16_t)(b >> 16) & 0x8000;
    int exp = (int)((b >> 23) & 0xff) - 127 + 15;
    uint32_t mant = b & 0x7fffff;
    if ((b & 0x7fffffff) > 0x7f800000) return sign | 0x7e00;
    if (exp >= 31) return sign | 0x7c00;
    if (exp <= 0) {
        if (exp < -10) return sign;
        mant |= 0x800000;
        unsigned shift = (unsigned)(14 - exp);
        uint32_t half = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half & 1))) half++;
        return sign | (uint16_t)half;
    }
    uint32_t half = ((uint32_t)exp << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (half & 1))) half++;
    return sign | (uint16_t)half;
}

/* q8gemm/gemm.go:329-341 f16ToF32: exact widening. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ff;
    if (exp == 0) {
        float s = sign ? -1.0f : 1.0f;
        return bitsf32(sign) + (float)mant * (1.0f / 16777216.0f) * s;
    }
    if (exp == 31) return bitsf32(sign | 0x7f800000 | (mant << 13));
    return bitsf32(sign | ((exp + 112) << 23) | (mant << 13));
}

/* q8gemm/packed.go:177 BF16ToF32. */
float orc_bf16_to_f32(uint16_t b) { return bitsf32((uint32_t)b << 16); }

/* q8gemm/gemm.go:138-150 MaxAbs: largest magnitude, or the first NaN met. */
float orc_max_abs(const float *x, int64_t n) {
    float m = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float v = x[i];
        if (v != v) return v;
        float a = bitsf32(f32bits(v) & 0x7fffffffu);
        if (a > m) m = a;
    }
    return m;
}

/* ------------------------------------------------------------------ */
/* q8gemv: fp32 activations x row-major int8 weights, one fp32 scale per row.
 * Pinned by: float64 products within the fp32 summation bound; exact answers
 * for the reference's own deterministic inputs (q8gemv_test.go:45-73); NaN
 * propagation (q8gemv_test.go:75-89); k = 0. */

/* q8gemv/scalar.go:8-17 scalarMulInto: sequential fp32 sum, then x scale. */
void orc_q8gemv_mul_into(const float *x, const int8_t *q, const float *scales, float *dst, int64_t k,
                         int64_t n) {
    for (int64_t row = 0; row < n; row++) {
        const int8_t *w = q + row * k;
        float sum = 0.0f;
        for (int64_t col = 0; col < k; col++) sum += x[col] * (float)w[col];
        dst[row] = sum * scales[row];
    }
}

/* Same loop with a fused multiply-add per step: the arm64 Go compiler fuses
 * `sum += x*w` (q8gemv/scalar.go:13 built for arm64). Brackets the two legal
 * scalar answers. */
void orc_q8gemv_mul_into_fma(const float *x, const int8_t *q, const float *scales, float *dst,
                             int64_t k, int64_t n) {
    for (int64_t row = 0; row < n; row++) {
        const int8_t *w = q + row * k;
        float sum = 0.0f;
        for (int64_t col = 0; col < k; col++) sum = fmaf(x[col], (float)w[col], sum);
        dst[row] = sum * scales[row];
    }
}

/* ------------------------------------------------------------------ */
/* qwen3lm GPU weight formats (block of 32 along K).
 * Pinned by: dequantize-and-compare bounds, code range, scale rounding
 * through numpy float16, brute-force scale search over the 16 candidates. */

/* qwen3lm/gpu_darwin.go:582-594 quantizeRow: s = max|row|/127, codes RNE of
 * v/s clamped to +-127. Returns s. */
float orc_quantize_row_q8(const float *row, int64_t k, int8_t *q) {
    float m = orc_max_abs(row, k);
    if (m == 0.0f) {
        memset(q, 0, (size_t)k);
        return 0.0f;
    }
    float s = m / 127.0f;
    for (int64_t i = 0; i < k; i++) {
        double r = nearbyint((double)(row[i] / s));
        if (r > 127) r = 127;
        if (r < -127) r = -127;
        q[i] = (int8_t)r;
    }
    return s;
}

/* qwen3lm/gpu_darwin.go:599-614 quantizeRowQ8B: per 32-block
 * d = f16(f16round(max/127)); codes RNE(x/d) clamped to +-127; stored scale
 * f16(d*mul). */
void orc_quantize_row_q8b(const float *row, int64_t k, int8_t *q, uint16_t *scales, float mul) {
    for (int64_t b = 0; b < k / 32; b++) {
        const float *v = row + b * 32;
        float d = orc_f16_to_f32(orc_f32_to_f16(orc_max_abs(v, 32) / 127.0f));
        scales[b] = orc_f32_to_f16(d * mul);
        if (d == 0.0f) {
            memset(q + b * 32, 0, 32);
            continue;
        }
        for (int i = 0; i < 32; i++) {
            double r = nearbyint((double)(v[i] / d));
            if (r > 127) r = 127;
            if (r < -127) r = -127;
            q[b * 32 + i] = (int8_t)r;
        }
    }
}

static inline float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }
static inline float abs32(float x) { return bitsf32(f32bits(x) & 0x7fffffffu); }

/* qwen3lm/gpu_darwin.go:616-658 quantizeRowQ4: per 32-block, 16 candidate
 * FP16 scales from peak/-8, squared error summed in fp32; value j in the low
 * nibble of byte j, value j+16 in the high nibble, both stored plus 8. */
void orc_quantize_row_q4(const float *row, int64_t k, uint8_t *dst, uint16_t *scales, float mul) {
    for (int64_t b = 0; b < k / 32; b++) {
        const float *v = row + b * 32;
        float peak = 0.0f;
        for (int i = 0; i < 32; i++)
            if (abs32(v[i]) > abs32(peak)) peak = v[i];
        float best = 0.0f, bestErr = INFINITY;
        if (peak != 0.0f) {
            for (int step = 0; step < 16; step++) {
                float d = peak / -8.0f * (1.0f - 0.02f * (float)step);
                d = orc_f16_to_f32(orc_f32_to_f16(d));
                if (d == 0.0f) continue;
                float e = 0.0f;
                for (int i = 0; i < 32; i++) {
                    float qv = clampf((float)nearbyint((double)(v[i] / d)), -8.0f, 7.0f);
                    float diff = v[i] - qv * d;
                    e += diff * diff;
                }
                if (e < bestErr) {
                    best = d;
                    bestErr = e;
                }
            }
        }
        uint8_t *out = dst + b * 16;
        for (int j = 0; j < 16; j++) {
            uint8_t lo = 8, hi = 8;
            if (best != 0.0f) {
                lo = (uint8_t)((int)clampf((float)nearbyint((double)(v[j] / best)), -8.0f, 7.0f) + 8);
                hi = (uint8_t)((int)clampf((float)nearbyint((double)(v[j + 16] / best)), -8.0f, 7.0f) + 8);
            }
            out[j] = (uint8_t)(lo | (hi << 4));
        }
        scales[b] = orc_f32_to_f16(best * mul);
    }
}

/* qwen3lm/gptq.go:762-791 q4GroupScale: the same 16-candidate search as
 * quantizeRowQ4, but the squared error is accumulated in float64. */
float orc_q4_group_scale(const float *v, int64_t len) {
    float peak = 0.0f;
    for (int64_t i = 0; i < len; i++)
        if (fabs((double)v[i]) > fabs((double)peak)) peak = v[i];
    if (peak == 0.0f) return 0.0f;
    float best = 0.0f;
    double bestErr = INFINITY;
    for (int step = 0; step < 16; step++) {
        float d = orc_f16_to_f32(orc_f32_to_f16(peak / -8.0f * (1.0f - 0.02f * (float)step)));
        if (d == 0.0f) continue;
        double e = 0.0;
        for (int64_t i = 0; i < len; i++) {
            double qv = nearbyint((double)(v[i] / d));
            if (qv > 7) qv = 7;
            if (qv < -8) qv = -8;
            double diff = (double)v[i] - qv * (double)d;
            e += diff * diff;
        }
        if (e < bestErr) {
            best = d;
            bestErr = e;
        }
    }
    return best;
}

/* ------------------------------------------------------------------ */
/* qwen3lm GEMV semantics (gpu.metal:68-162), restated as scalar loops. The
 * Metal kernel sums lanes with simd_sum, whose order is unspecified, so these
 * restatements are tolerance references (the float64 functions below are the
 * bound), not bit-exact targets.
 *
 * fmt: 8 = Q8 (int8 codes, fp32 scale per row), 9 = Q8B (int8 codes, f16 scale
 * per 32), 10 = Q8 with fp32 scale per 32 (the benchmark config-1 variant),
 * 4 = Q4 (split nibbles, f16 scale per 32). */

static float scale_of(int fmt, const void *scale, int64_t row, int64_t k, int64_t i) {
    if (fmt == 9 || fmt == 4) return orc_f16_to_f32(((const uint16_t *)scale)[row * (k / 32) + i / 32]);
    if (fmt == 10) return ((const float *)scale)[row * (k / 32) + i / 32];
    return 1.0f;
}

/* gpu.metal:85-123: 16-value chunks for 8-bit codes (t = sum of 4 dot4s, then
 * acc = fma(d, t, acc) for block scales, acc += t for Q8); 32-value blocks for
 * Q4 (acc = fma(d, sum(nib*x) - 8*sum(x), acc)); chunks visited in increasing
 * K; gpu.metal:126-129 then scales Q8 rows by their fp32 scale. */
void orc_gemv(int fmt, const void *codes, const void *scale, const float *x, float *y, int64_t k,
              int64_t n) {
    for (int64_t row = 0; row < n; row++) {
        float acc = 0.0f;
        if (fmt != 4) {
            const int8_t *w = (const int8_t *)codes + row * k;
            for (int64_t i = 0; i < k; i += 16) {
                float d4[4];
                for (int c = 0; c < 4; c++) {
                    const int8_t *wc = w + i + 4 * c;
                    const float *xc = x + i + 4 * c;
                    d4[c] = (float)wc[0] * xc[0] + (float)wc[1] * xc[1] + (float)wc[2] * xc[2] +
                            (float)wc[3] * xc[3];
                }
                float t = d4[0] + d4[1] + d4[2] + d4[3];
                if (fmt == 8)
                    acc += t;
                else
                    acc = fmaf(scale_of(fmt, scale, row, k, i), t, acc);
            }
            if (fmt == 8) acc *= ((const float *)scale)[row];
        } else {
            const uint8_t *w = (const uint8_t *)codes + row * (k / 2);
            for (int64_t i = 0; i < k; i += 32) {
                const uint8_t *b = w + i / 2;
                float sx = 0.0f, t = 0.0f;
                for (int j = 0; j < 32; j++) sx += x[i + j];
                sx *= 8.0f;
                for (int j = 0; j < 16; j++) {
                    t = fmaf((float)(b[j] & 15), x[i + j], t);
                    t = fmaf((float)(b[j] >> 4), x[i + 16 + j], t);
                }
                acc = fmaf(scale_of(fmt, scale, row, k, i), t - sx, acc);
            }
        }
        y[row] = acc;
    }
}

/* Dequantized weight value of a qwen3lm GPU format: the float64 reference the
 * reference GPU tests use (gpu_darwin_test.go:44-56, 203-212). */
double orc_dequant(int fmt, const void *codes, const void *scale, int64_t row, int64_t k, int64_t i) {
    if (fmt == 4) {
        uint8_t b = ((const uint8_t *)codes)[row * (k / 2) + (i / 32) * 16 + i % 16];
        int q = (i % 32 >= 16) ? (int)(b >> 4) - 8 : (int)(b & 15) - 8;
        return (double)q * (double)scale_of(fmt, scale, row, k, i);
    }
    double c = (double)((const int8_t *)codes)[row * k + i];
    if (fmt == 8) return c * (double)((const float *)scale)[row];
    return c * (double)scale_of(fmt, scale, row, k, i);
}

/* float64 y = W_dequant . x, and sum |w x| for error bounds. */
void orc_gemv_f64(int fmt, const void *codes, const void *scale, const float *x, double *y,
                  double *abs_sum, int64_t k, int64_t n) {
    for (int64_t row = 0; row < n; row++) {
        double s = 0.0, a = 0.0;
        for (int64_t i = 0; i < k; i++) {
            double p = orc_dequant(fmt, codes, scale, row, k, i) * (double)x[i];
            s += p;
            a += fabs(p);
        }
        y[row] = s;
        if (abs_sum) abs_sum[row] = a;
    }
}

/* ------------------------------------------------------------------ */
/* q8gemm F16 path.
 * Pinned by: frexp property max*scale in [2^14, 2^15) (Python math.frexp);
 * numpy float16 conversion of every packed value; the reference's own
 * float64 error bound (1/2048 + 1e-5) * sum|x w| * scale (q8gemm_test.go:81);
 * BF16 packing exactness (q8gemm_test.go:290-352). */

/* q8gemm/gemm.go:127-135 SetRowScale: e = clamp(15 - exp(max), -100, 100)
 * when max is finite and positive, else 0; scale 2^e, inverse 2^-e. */
void orc_f16_row_scale(float max_abs, float *scale, float *inverse) {
    int e = 0;
    if (max_abs > 0 && !isinf(max_abs) && !isnan(max_abs)) {
        int exp;
        frexp((double)max_abs, &exp);
        e = 15 - exp;
        if (e < -100) e = -100;
        if (e > 100) e = 100;
    }
    *scale = (float)ldexp(1.0, e);
    *inverse = (float)ldexp(1.0, -e);
}

/* q8gemm/gemm.go:65-77 Workspace.Pack + gemm.go:155-226 PackRange (general
 * tile): every value becomes f32ToF16(x * rowScale). Output is logical
 * [rows][k] FP16 bits plus each row's scale and inverse. */
void orc_f16_pack_rows(const float *x, int64_t rows, int64_t k, int64_t stride, uint16_t *out,
                       float *row_scale, float *row_inverse) {
    for (int64_t r = 0; r < rows; r++) {
        float s, inv;
        orc_f16_row_scale(orc_max_abs(x + r * stride, k), &s, &inv);
        row_scale[r] = s;
        row_inverse[r] = inv;
        for (int64_t i = 0; i < k; i++) out[r * k + i] = orc_f32_to_f16(x[r * stride + i] * s);
    }
}

/* q8gemm/packed.go:128-175 PackBF16Rows for one row: power-of-two shift of
 * the row into [2^14, 2^15), FP16 conversion, count of rounded values.
 * Returns -1 for a non-finite weight (ErrNonFinite), else the rounded count.
 * out is the row's logical FP16 values; *row_scale the stored inverse. */
int64_t orc_pack_bf16_row(const uint16_t *bf16, int64_t k, uint16_t *out, float *row_scale) {
    float maxAbs = 0.0f;
    for (int64_t i = 0; i < k; i++) {
        float v = orc_bf16_to_f32(bf16[i]);
        if (isnan(v) || isinf(v)) return -1;
        float a = fabsf(v);
        if (a > maxAbs) maxAbs = a;
    }
    int e = 0;
    if (maxAbs > 0) {
        int exp;
        frexp((double)maxAbs, &exp);
        e = 15 - exp;
        if (e < -100) e = -100;
        if (e > 100) e = 100;
    }
    float scale = (float)ldexp(1.0, e);
    *row_scale = (float)ldexp(1.0, -e);
    int64_t rounded = 0;
    for (int64_t i = 0; i < k; i++) {
        float v = orc_bf16_to_f32(bf16[i]) * scale;
        uint16_t h = orc_f32_to_f16(v);
        if (orc_f16_to_f32(h) != v) rounded++;
        out[i] = h;
    }
    return rounded;
}

/* q8gemm/scalar.go:9-20 scalarMulPanels (== portable.go:20-66 on amd64: the
 * same products, summed in increasing K in fp32 with no fusion):
 * dst[r*stride+c] = (sum_k f16(a[r,k]) * w[c,k]) * scales[c] * rowInverse[r]
 * for columns [p0*64, min(p1*64, n)). w is int8 (w_f16 == NULL) or FP16. */
void orc_mul_panels(float *dst, int64_t stride, const uint16_t *act, const float *row_inverse,
                    int64_t rows, const int8_t *w_i8, const uint16_t *w_f16, const float *scales,
                    int64_t k, int64_t n, int64_t p0, int64_t p1) {
    int64_t c1 = p1 * OUTPUT_PANEL < n ? p1 * OUTPUT_PANEL : n;
    for (int64_t col = p0 * OUTPUT_PANEL; col < c1; col++) {
        for (int64_t r = 0; r < rows; r++) {
            float sum = 0.0f;
            for (int64_t i = 0; i < k; i++) {
                float a = orc_f16_to_f32(act[r * k + i]);
                float w = w_f16 ? orc_f16_to_f32(w_f16[col * k + i]) : (float)w_i8[col * k + i];
                sum += a * w;
            }
            dst[r * stride + col] = sum * scales[col] * row_inverse[r];
        }
    }
}

/* q8gemm/packed.go:183-204 Weights.Pack layout [panel][K/2][64][2] (and
 * packed.go:162-171 for FP16): element (row, k) lands at index
 * panel*pairs*128 + (k/2)*128 + (row%64)*2 + k%2 (packed.go:233-239 at()). */
void orc_pack_panels_u16(const uint16_t *src, int64_t k, int64_t n, uint16_t *out) {
    int64_t pairs = (k + 1) / 2, panels = (n + OUTPUT_PANEL - 1) / OUTPUT_PANEL;
    memset(out, 0, (size_t)(panels * pairs * 2 * OUTPUT_PANEL) * 2);
    for (int64_t row = 0; row < n; row++)
        for (int64_t i = 0; i < k; i++)
            out[(row / OUTPUT_PANEL) * pairs * 2 * OUTPUT_PANEL + (i / 2) * 2 * OUTPUT_PANEL +
                (row % OUTPUT_PANEL) * 2 + i % 2] = src[row * k + i];
}

void orc_pack_panels_i8(const int8_t *src, int64_t k, int64_t n, int8_t *out) {
    int64_t pairs = (k + 1) / 2, panels = (n + OUTPUT_PANEL - 1) / OUTPUT_PANEL;
    memset(out, 0, (size_t)(panels * pairs * 2 * OUTPUT_PANEL));
    for (int64_t row = 0; row < n; row++)
        for (int64_t i = 0; i < k; i++)
            out[(row / OUTPUT_PANEL) * pairs * 2 * OUTPUT_PANEL + (i / 2) * 2 * OUTPUT_PANEL +
                (row % OUTPUT_PANEL) * 2 + i % 2] = src[row * k + i];
}

/* ------------------------------------------------------------------ */
/* q8gemm int8 x int8 path.
 * Pinned by: numpy (x * inv rounded with np.rint, clipped) for the quantizer;
 * exact int64 matmul (numpy) for the integer sums; the reference's float64
 * bound 0.5 * rowScale * sum|w| (int8_test.go:83-96). */

/* q8gemm/int8.go:106-112 SetRowScale: max/127 and 127/max when max is
 * finite and positive, else 0 and 0. */
void orc_i8_row_scale(float max_abs, float *scale, float *inverse) {
    if (max_abs > 0 && !isinf(max_abs) && max_abs == max_abs) {
        *scale = max_abs / 127.0f;
        *inverse = 127.0f / max_abs;
        return;
    }
    *scale = 0.0f;
    *inverse = 0.0f;
}

/* q8gemm/int8.go:163-168 quantize: round half to even, saturate to int8. A NaN
 * (x * 0 for a non-finite row) converts to 0, which is what Go's float->int8
 * conversion yields on amd64 (CVTTSD2SL -> 0x80000000, low byte 0) and arm64
 * (FCVTZS NaN -> 0). */
int8_t orc_i8_quantize(float v) {
    if (v != v) return 0;
    double r = nearbyint((double)v);
    if (r > 127) r = 127;
    if (r < -128) r = -128;
    return (int8_t)r;
}

/* q8gemm/int8.go:116-163 PackRange over a whole prepared tile after
 * SetRowScale(MaxAbs(row)) (int8_test.go:32-43 packI8): logical [rows][k]
 * codes plus each row's scale and inverse. */
void orc_i8_pack_rows(const float *x, int64_t rows, int64_t k, int64_t stride, int8_t *out,
                      float *row_scale, float *row_inverse) {
    for (int64_t r = 0; r < rows; r++) {
        float s, inv;
        orc_i8_row_scale(orc_max_abs(x + r * stride, k), &s, &inv);
        row_scale[r] = s;
        row_inverse[r] = inv;
        for (int64_t i = 0; i < k; i++) out[r * k + i] = orc_i8_quantize(x[r * stride + i] * inv);
    }
}

/* q8gemm/int8.go:200-211 scalarMulPanelsI8: exact int32 sum, then
 * float32(sum) * scales[col] * rowScale[row], left to right. */
void orc_i8_mul_panels(float *dst, int64_t stride, const int8_t *act, const float *row_scale,
                       int64_t rows, const int8_t *w, const float *scales, int64_t k, int64_t n,
                       int64_t p0, int64_t p1) {
    int64_t c1 = p1 * OUTPUT_PANEL < n ? p1 * OUTPUT_PANEL : n;
    for (int64_t col = p0 * OUTPUT_PANEL; col < c1; col++) {
        for (int64_t r = 0; r < rows; r++) {
            int32_t sum = 0;
            for (int64_t i = 0; i < k; i++) sum += (int32_t)act[r * k + i] * (int32_t)w[col * k + i];
            dst[r * stride + col] = (float)sum * scales[col] * row_scale[r];
        }
    }
}

/* Block-32 int8 variant (benchmark configuration 2's wording; the reference's
 * q8gemm int8 path scales per row): every 32-value block of a row takes the
 * per-row rule of WorkspaceI8 (int8.go:106-119: scale max/127, inverse 127/max,
 * both 0 unless 0 < max < inf) and quantize's codes (int8.go:163-168). q is
 * [rows][k], d is [rows][k/32]. No counterpart function in the reference. */
void orc_q8b_quantize(const float *x, int64_t rows, int64_t k, int64_t stride, int8_t *q, float *d) {
    const int64_t kb = k / 32;
    for (int64_t r = 0; r < rows; r++)
        for (int64_t b = 0; b < kb; b++) {
            float s, inv;
            const float *xb = x + r * stride + b * 32;
            orc_i8_row_scale(orc_max_abs(xb, 32), &s, &inv);
            d[r * kb + b] = s;
            for (int i = 0; i < 32; i++) q[r * k + b * 32 + i] = orc_i8_quantize(xb[i] * inv);
        }
}

/* Block-32 int8 GEMM: for each output, over the 32-value blocks b in
 * increasing order, acc = fmaf((float)dot_b, da[r][b] * dw[c][b], acc) with
 * dot_b the exact int32 block product and acc starting at +0.0f. Activations
 * qa [m][k] with scales da [m][k/32]; weights qw [n][k] (row-major, as the
 * GPU formats) with scales dw [n][k/32]; y [m][n]. */
void orc_q8b_gemm(const int8_t *qa, const float *da, const int8_t *qw, const float *dw, float *y, int64_t m,
                  int64_t k, int64_t n) {
    const int64_t kb = k / 32;
    for (int64_t r = 0; r < m; r++)
        for (int64_t c = 0; c < n; c++) {
            float acc = 0.0f;
            for (int64_t b = 0; b < kb; b++) {
                int32_t dot = 0;
                for (int i = 0; i < 32; i++)
                    dot += (int32_t)qa[r * k + b * 32 + i] * (int32_t)qw[c * k + b * 32 + i];
                const float s = da[r * kb + b] * dw[c * kb + b];
                acc = fmaf((float)dot, s, acc);
            }
            y[r * n + c] = acc;
        }
}

/* Multi-threaded restatement of the same oracle for the CPU baseline: the
 * reference splits 64-column panels across its worker pool
 * (qwen3lm/ops.go:153-214); the arithmetic per output is identical. */
#include <pthread.h>
typedef struct {
    float *dst;
    int64_t stride;
    const int8_t *act;
    const float *row_scale;
    int64_t rows;
    const int8_t *w;
    const float *scales;
    int64_t k, n, p0, p1;
} i8_job;

static void *i8_worker(void *arg) {
    i8_job *j = (i8_job *)arg;
    orc_i8_mul_panels(j->dst, j->stride, j->act, j->row_scale, j->rows, j->w, j->scales, j->k, j->n,
                      j->p0, j->p1);
    return 0;
}

void orc_i8_mul_panels_mt(float *dst, int64_t stride, const int8_t *act, const float *row_scale,
                          int64_t rows, const int8_t *w, const float *scales, int64_t k, int64_t n,
                          int threads) {
    int64_t panels = (n + OUTPUT_PANEL - 1) / OUTPUT_PANEL;
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t tid[64];
    i8_job jobs[64];
    for (int t = 0; t < threads; t++) {
        int64_t a = panels * t / threads, b = panels * (t + 1) / threads;
        jobs[t] = (i8_job){dst, stride, act, row_scale, rows, w, scales, k, n, a, b};
        pthread_create(&tid[t], 0, i8_worker, &jobs[t]);
    }
    for (int t = 0; t < threads; t++) pthread_join(tid[t], 0);
}

/* q8gemm/int8.go:53-77 WeightsI8 layout [panel][K/4][64][4]: element
 * (row, k) at panel*quads*256 + (k/4)*256 + (row%64)*4 + k%4. */
void orc_pack_panels_i8_quads(const int8_t *src, int64_t k, int64_t n, int8_t *out) {
    int64_t quads = (k + 3) / 4, panels = (n + OUTPUT_PANEL - 1) / OUTPUT_PANEL;
    memset(out, 0, (size_t)(panels * quads * 4 * OUTPUT_PANEL));
    for (int64_t row = 0; row < n; row++)
        for (int64_t i = 0; i < k; i++)
            out[(row / OUTPUT_PANEL) * quads * 4 * OUTPUT_PANEL + (i / 4) * 4 * OUTPUT_PANEL +
                (row % OUTPUT_PANEL) * 4 + i % 4] = src[row * k + i];
}

/* Array forms of the conversions above (same arithmetic, one call). */
void orc_f32_to_f16_array(const float *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = orc_f32_to_f16(src[i]);
}

void orc_f16_to_f32_array(const uint16_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32(src[i]);
}

void orc_i8_quantize_array(const float *src, int8_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = orc_i8_quantize(src[i]);
}

/* ------------------------------------------------------------------ */
/* qwen3lm mm semantics (gpu.metal:766-927, PRO_PLAIN / EPI_STORE) and the
 * group-128 zero-point int4 variant. Each K step's weight tile is FP16:
 * Q8 half(code) (exact), Q8B half(code)*half(d) and Q4 (half(nib)-8)*d,
 * rounded to half (gpu.metal:836-861); activations half(x) (gpu.metal:
 * 828-829, 863-865 with inv = 1). Products of two halves are exact in fp32 and
 * float64; the sum here is float64 (the bound reference), and Q8 rows are
 * then scaled by their fp32 scale (gpu.metal:898-899).
 * fmt 12 (GPTQ4_G128): codes u32 [n][k/8], nibble i of word j = k 8j+i;
 * scales f16 [n][k/128]; zeros u8 [n][k/128]; w = half((q - z) * s).
 * Pinned by: the dequantization rule of gpu_darwin_test.go:44-56 (Q4) and
 * exact float64 products; numpy float16 rounding in tests/test_oracle.py. */
static float mm_weight(int fmt, const void *codes, const void *scales, const uint8_t *zeros, int64_t row,
                       int64_t k, int64_t i) {
    if (fmt == 8) return (float)((const int8_t *)codes)[row * k + i];
    if (fmt == 9) {
        float d = orc_f16_to_f32(((const uint16_t *)scales)[row * (k / 32) + i / 32]);
        float c = (float)((const int8_t *)codes)[row * k + i];
        return orc_f16_to_f32(orc_f32_to_f16(c * d));
    }
    if (fmt == 10) { /* Q8B with fp32 block scales: half(code) * half(d), rounded to half */
        float d = orc_f16_to_f32(orc_f32_to_f16(((const float *)scales)[row * (k / 32) + i / 32]));
        float c = (float)((const int8_t *)codes)[row * k + i];
        return orc_f16_to_f32(orc_f32_to_f16(c * d));
    }
    if (fmt == 4) {
        uint8_t b = ((const uint8_t *)codes)[row * (k / 2) + (i / 32) * 16 + i % 16];
        int q = (i % 32 >= 16) ? (int)(b >> 4) : (int)(b & 15);
        float d = orc_f16_to_f32(((const uint16_t *)scales)[row * (k / 32) + i / 32]);
        return orc_f16_to_f32(orc_f32_to_f16((float)(q - 8) * d));
    }
    /* fmt 12 */
    uint32_t wd = ((const uint32_t *)codes)[row * (k / 8) + i / 8];
    int q = (int)((wd >> (4 * (i % 8))) & 15);
    int z = zeros[row * (k / 128) + i / 128] & 15;
    float s = orc_f16_to_f32(((const uint16_t *)scales)[row * (k / 128) + i / 128]);
    return orc_f16_to_f32(orc_f32_to_f16((float)(q - z) * s));
}

void orc_mm_f64(int fmt, const void *codes, const void *scales, const uint8_t *zeros, const float *x, double *y,
                double *abs_sum, int64_t m, int64_t k, int64_t n) {
    for (int64_t c = 0; c < n; c++) {
        for (int64_t r = 0; r < m; r++) {
            double s = 0.0, a = 0.0;
            for (int64_t i = 0; i < k; i++) {
                double p = (double)orc_f16_to_f32(orc_f32_to_f16(x[r * k + i])) *
                           (double)mm_weight(fmt, codes, scales, zeros, c, k, i);
                s += p;
                a += fabs(p);
            }
            if (fmt == 8) {
                double sc = (double)((const float *)scales)[c];
                s *= sc;
                a *= fabs(sc);
            }
            y[r * n + c] = s;
            if (abs_sum) abs_sum[r * n + c] = a;
        }
    }
}

/* The group-128 zero-point int4 weights without FP16 rounding, (q - z) * s in
 * float64: the "true" dequantized matrix the 2e-3 tolerance refers to. */
double orc_gptq_g128_weight(const uint32_t *codes, const uint16_t *scales, const uint8_t *zeros, int64_t row,
                            int64_t k, int64_t i) {
    uint32_t wd = codes[row * (k / 8) + i / 8];
    int q = (int)((wd >> (4 * (i % 8))) & 15);
    int z = zeros[row * (k / 128) + i / 128] & 15;
    return (double)(q - z) * (double)orc_f16_to_f32(scales[row * (k / 128) + i / 128]);
}

/* ------------------------------------------------------------------ */
/* Randomized Hadamard rotation of the qwen3lm GPU residual stream.
 * Pinned by: splitmix64 against its published first outputs; apply against
 * the dense matrix scale*H*diag(signs) (scipy's Sylvester Hadamard) in
 * float64; orthogonality and dot-product preservation as
 * qwen3lm/kernels_test.go:73-111; unapply(apply(x)) == x (tests/test_oracle_lm.py). */

/* One splitmix64 step (Steele, Lea and Flood 2014), as hadamard.go:33-38:
 * state += golden; z = state; two xor-shift-multiply rounds; z ^= z >> 31. */
uint64_t orc_splitmix64_next(uint64_t *state) {
    *state += 0x9e3779b97f4a7c15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* hadamard.go:24-47 newRotation: block is the largest power of two up to
 * 4096 dividing k; sign i is -1 when the low bit of the i-th splitmix64
 * output (state seeded with golden ^ k) is set; scale = float32(1/sqrt(block)).
 * Returns the block; writes k signs and the scale. */
int64_t orc_rotation(int64_t k, float *signs, float *scale) {
    int64_t block = 1;
    while (block < 4096 && k % (2 * block) == 0) block *= 2;
    uint64_t state = 0x9e3779b97f4a7c15ull ^ (uint64_t)k;
    for (int64_t i = 0; i < k; ++i) signs[i] = (orc_splitmix64_next(&state) & 1) ? -1.0f : 1.0f;
    *scale = (float)(1.0 / sqrt((double)block));
    return block;
}

/* hadamard.go:62-78 fwht: the unnormalized Walsh-Hadamard butterfly network
 * in natural (Sylvester) order, stage h = 1, 2, 4, ...: (a, b) -> (a+b, a-b). */
void orc_fwht(float *v, int64_t n) {
    for (int64_t h = 1; h < n; h *= 2)
        for (int64_t i = 0; i < n; i += 2 * h)
            for (int64_t j = i; j < i + h; ++j) {
                float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
}

/* hadamard.go:51-58 apply: per block, v = (v * scale) * sign, then fwht. */
void orc_rotation_apply(const float *signs, int64_t block, float scale, float *x, int64_t k) {
    for (int64_t b = 0; b < k; b += block) {
        for (int64_t i = b; i < b + block; ++i) x[i] = x[i] * scale * signs[i];
        orc_fwht(x + b, block);
    }
}

/* hadamard.go:80-86 unapply: fwht per block, then (v * scale) * sign. */
void orc_rotation_unapply(const float *signs, int64_t block, float scale, float *x, int64_t k) {
    for (int64_t b = 0; b < k; b += block) orc_fwht(x + b, block);
    for (int64_t i = 0; i < k; ++i) x[i] = x[i] * scale * signs[i];
}

/* hadamard.go:88-104 applyRows: the n x k matrix a becomes R.a, rotating along
 * the row index: each row times its sign, the butterfly network across rows
 * of each block (stage h = 1, 2, ...), then every value times scale. */
void orc_rotation_apply_rows(const float *signs, int64_t block, float scale, float *a, int64_t n, int64_t k) {
    for (int64_t i = 0; i < n; ++i)
        for (int64_t c = 0; c < k; ++c) a[i * k + c] *= signs[i];
    for (int64_t b = 0; b < n; b += block)
        for (int64_t h = 1; h < block; h *= 2)
            for (int64_t i = b; i < b + block; i += 2 * h)
                for (int64_t j = i; j < i + h; ++j)
                    for (int64_t c = 0; c < k; ++c) {
                        float x = a[j * k + c], y = a[(j + h) * k + c];
                        a[j * k + c] = x + y;
                        a[(j + h) * k + c] = x - y;
                    }
    for (int64_t i = 0; i < n * k; ++i) a[i] *= scale;
}

/* One gpuJob of prepareGPU (qwen3lm/gpu_darwin.go:511-567) on the CPU: rows of
 * BF16 bits [n][k] widened to float32; each row times the folded norm (if
 * any), then rotated by the input rotation (if any); then the output rotation
 * along the rows (if any); then each row quantized in format fmt (8 = Q8 with
 * an fp32 row scale times scale_mul, 9 = Q8B, 4 = Q4, 10 = Q8B with fp32 block
 * scales) into dst at byte offsets base (codes) and sc (scales), source row r
 * landing on destination row row0 + r*step. in_signs/out_signs may be NULL. */
void orc_prepare_projection(const uint16_t *bf16, int64_t n, int64_t k, const float *norm, const float *in_signs,
                            int64_t in_block, float in_scale, const float *out_signs, int64_t out_block,
                            float out_scale, int fmt, uint8_t *dst, int64_t base, int64_t sc, int64_t step,
                            int64_t row0, float scale_mul, float *work) {
    for (int64_t i = 0; i < n * k; ++i) work[i] = orc_bf16_to_f32(bf16[i]);
    for (int64_t r = 0; r < n; ++r) {
        float *row = work + r * k;
        if (norm)
            for (int64_t i = 0; i < k; ++i) row[i] *= norm[i];
        if (in_signs) orc_rotation_apply(in_signs, in_block, in_scale, row, k);
    }
    if (out_signs) orc_rotation_apply_rows(out_signs, out_block, out_scale, work, n, k);
    for (int64_t r = 0; r < n; ++r) {
        const float *row = work + r * k;
        const int64_t d = row0 + r * step;
        if (fmt == 8) {
            float s = orc_quantize_row_q8(row, k, (int8_t *)(dst + base + d * k));
            float v = s * scale_mul;
            memcpy(dst + sc + d * 4, &v, 4);
        } else if (fmt == 9) {
            orc_quantize_row_q8b(row, k, (int8_t *)(dst + base + d * k), (uint16_t *)(dst + sc + d * (k / 32) * 2),
                                 scale_mul);
        } else if (fmt == 4) {
            orc_quantize_row_q4(row, k, dst + base + d * (k / 2), (uint16_t *)(dst + sc + d * (k / 32) * 2),
                                scale_mul);
        } else if (fmt == 10) {
            int8_t *q = (int8_t *)(dst + base + d * k);
            float *s = (float *)(dst + sc + d * (k / 32) * 4);
            for (int64_t b = 0; b < k / 32; b++) {
                float dd = orc_max_abs(row + b * 32, 32) / 127.0f;
                s[b] = dd * scale_mul;
                for (int i = 0; i < 32; i++) {
                    double q0 = dd == 0.0f ? 0.0 : nearbyint((double)(row[b * 32 + i] / dd));
                    if (q0 > 127) q0 = 127;
                    if (q0 < -127) q0 = -127;
                    q[b * 32 + i] = (int8_t)q0;
                }
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* CPU decode step for the CPU baseline (bench.py cpu_baseline): one token of
 * a dense Qwen3 through the reference's CPU int8 path (qwen3lm/ops.go:96-254
 * with WeightsInt8, weights.go:314-349): the residual unrotated; per
 * projection input, RMSNorm with its weight (rmsNorm32), the int8
 * projections' input rotation (ops.go:110-122: newRotation of the hidden
 * width for q/k/v/gate/up and the head, of q_dim for o, of the intermediate
 * width for down), per-row int8 quantization (int8.go:106-168) and
 * scalarMulPanelsI8 (int8.go:200-211) split over 64-column panels across T
 * workers (ops.go:153-214); head RMSNorm + RoPE, softmax attention over the
 * fp32 K/V cache, SwiGLU, residual adds; final norm and the int8 head. The
 * workers meet at a barrier between stages, as the reference's pool does.
 * Pinned to the float64 CpuInt8Oracle (oracle/lm_oracle.py), itself pinned to
 * the GPU-basis decode oracle, in tests/test_cpu_baseline.py. */

typedef struct {
    int64_t hidden, heads, kv_heads, head_dim, inter, vocab, layers, cap;
    float eps;
} orc_lm_geom;

typedef struct {
    const int8_t *w[7];      /* q, k, v, o, gate, up, down: [n][k] */
    const float *s[7];       /* per-row scales */
    const float *attn_norm, *mlp_norm, *q_norm, *k_norm;
} orc_lm_layer_i8;

typedef struct {
    const orc_lm_geom *g;
    const orc_lm_layer_i8 *L;
    float *kc, *vc;          /* [layers][cap][kvd] */
    const float *cosv, *sinv; /* [head_dim/2] at this position */
    const float *final_norm;
    const int8_t *head;
    const float *head_s;
    float *h, *x, *qkv, *ctx, *tmp, *act, *logits, *scores;
    int8_t *qa;
    float rs;
    int pos, threads;
    /* The int8 projections' input rotations (weights.go:314-316): newRotation
     * of the hidden width, of the attention context (q_dim) and of the
     * intermediate width. */
    float *rot_h, *rot_c, *rot_i;
    int64_t blk_h, blk_c, blk_i;
    float sc_h, sc_c, sc_i;
    pthread_barrier_t bar;
} lm_step_ctx;

static void rms_norm32(float *out, const float *x, const float *w, int64_t n, float eps) {
    /* kernels_scalar.go sumSquares in float64, then float32 scaling (ops.go:251-254). */
    double ss = 0;
    for (int64_t i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float inv = (float)(1.0 / sqrt(ss / (double)n + eps));
    for (int64_t i = 0; i < n; i++) out[i] = x[i] * inv * (w ? w[i] : 1.0f);
}

static void quantize_row(lm_step_ctx *c, const float *x, int64_t k) {
    float s, inv;
    orc_i8_row_scale(orc_max_abs(x, k), &s, &inv);
    c->rs = s;
    for (int64_t i = 0; i < k; i++) c->qa[i] = orc_i8_quantize(x[i] * inv);
}

/* This worker's share of panels of an n x k int8 projection of c->qa. */
static void project_share(lm_step_ctx *c, int t, const int8_t *w, const float *s, int64_t k, int64_t n, float *y) {
    const int64_t panels = (n + OUTPUT_PANEL - 1) / OUTPUT_PANEL;
    const int64_t p0 = panels * t / c->threads, p1 = panels * (t + 1) / c->threads;
    orc_i8_mul_panels(y, n, c->qa, &c->rs, 1, w, s, k, n, p0, p1);
}

typedef struct {
    lm_step_ctx *c;
    int t;
} lm_worker;

static void *lm_step_worker(void *arg) {
    lm_step_ctx *c = ((lm_worker *)arg)->c;
    const int t = ((lm_worker *)arg)->t;
    const orc_lm_geom *g = c->g;
    const int64_t H = g->hidden, hd = g->head_dim, qd = g->heads * hd, kvd = g->kv_heads * hd, I = g->inter;
    const int64_t grp = g->heads / g->kv_heads, n = c->pos + 1;
    for (int64_t l = 0; l < g->layers; l++) {
        const orc_lm_layer_i8 *L = &c->L[l];
        float *kc = c->kc + l * g->cap * kvd, *vc = c->vc + l * g->cap * kvd;
        if (t == 0) {
            rms_norm32(c->x, c->h, L->attn_norm, H, g->eps);
            orc_rotation_apply(c->rot_h, c->blk_h, c->sc_h, c->x, H);
            quantize_row(c, c->x, H);
        }
        pthread_barrier_wait(&c->bar);
        project_share(c, t, L->w[0], L->s[0], H, qd, c->qkv);
        project_share(c, t, L->w[1], L->s[1], H, kvd, c->qkv + qd);
        project_share(c, t, L->w[2], L->s[2], H, kvd, c->qkv + qd + kvd);
        pthread_barrier_wait(&c->bar);
        /* K/V append, then attention per query head (heads split over workers). */
        if (t == 0) {
            for (int64_t kh = 0; kh < g->kv_heads; kh++) {
                float *kr = c->qkv + qd + kh * hd;
                rms_norm32(kr, kr, L->k_norm, hd, g->eps);
                for (int64_t d = 0; d < hd / 2; d++) {
                    const float a = kr[d], b = kr[d + hd / 2];
                    kr[d] = a * c->cosv[d] - b * c->sinv[d];
                    kr[d + hd / 2] = b * c->cosv[d] + a * c->sinv[d];
                }
                memcpy(kc + c->pos * kvd + kh * hd, kr, hd * 4);
                memcpy(vc + c->pos * kvd + kh * hd, c->qkv + qd + kvd + kh * hd, hd * 4);
            }
        }
        pthread_barrier_wait(&c->bar);
        for (int64_t qh = t; qh < g->heads; qh += c->threads) {
            float *q = c->qkv + qh * hd;
            rms_norm32(q, q, L->q_norm, hd, g->eps);
            for (int64_t d = 0; d < hd / 2; d++) {
                const float a = q[d], b = q[d + hd / 2];
                q[d] = a * c->cosv[d] - b * c->sinv[d];
                q[d + hd / 2] = b * c->cosv[d] + a * c->sinv[d];
            }
            const int64_t kh = qh / grp;
            float *sc = c->scores + t * g->cap;
            float mx = -INFINITY;
            const float scale = (float)(1.0 / sqrt((double)hd));
            for (int64_t j = 0; j < n; j++) {
                float s = 0;
                for (int64_t d = 0; d < hd; d++) s += q[d] * kc[j * kvd + kh * hd + d];
                sc[j] = s * scale;
                mx = sc[j] > mx ? sc[j] : mx;
            }
            float sum = 0;
            for (int64_t j = 0; j < n; j++) sum += (sc[j] = expf(sc[j] - mx));
            float *o = c->ctx + qh * hd;
            for (int64_t d = 0; d < hd; d++) o[d] = 0;
            for (int64_t j = 0; j < n; j++) {
                const float p = sc[j] / sum;
                for (int64_t d = 0; d < hd; d++) o[d] += p * vc[j * kvd + kh * hd + d];
            }
        }
        pthread_barrier_wait(&c->bar);
        if (t == 0) {
            memcpy(c->x, c->ctx, qd * 4);
            orc_rotation_apply(c->rot_c, c->blk_c, c->sc_c, c->x, qd);
            quantize_row(c, c->x, qd);
        }
        pthread_barrier_wait(&c->bar);
        project_share(c, t, L->w[3], L->s[3], qd, H, c->tmp);
        pthread_barrier_wait(&c->bar);
        if (t == 0) {
            for (int64_t i = 0; i < H; i++) c->h[i] += c->tmp[i];
            rms_norm32(c->x, c->h, L->mlp_norm, H, g->eps);
            orc_rotation_apply(c->rot_h, c->blk_h, c->sc_h, c->x, H);
            quantize_row(c, c->x, H);
        }
        pthread_barrier_wait(&c->bar);
        project_share(c, t, L->w[4], L->s[4], H, I, c->act);
        project_share(c, t, L->w[5], L->s[5], H, I, c->act + I);
        pthread_barrier_wait(&c->bar);
        if (t == 0) {
            for (int64_t i = 0; i < I; i++) {
                const float gt = c->act[i], up = c->act[I + i];
                c->act[i] = gt / (1.0f + expf(-gt)) * up;
            }
            orc_rotation_apply(c->rot_i, c->blk_i, c->sc_i, c->act, I);
            quantize_row(c, c->act, I);
        }
        pthread_barrier_wait(&c->bar);
        project_share(c, t, L->w[6], L->s[6], I, H, c->tmp);
        pthread_barrier_wait(&c->bar);
        if (t == 0)
            for (int64_t i = 0; i < H; i++) c->h[i] += c->tmp[i];
    }
    if (t == 0) {
        rms_norm32(c->x, c->h, c->final_norm, H, g->eps);
        orc_rotation_apply(c->rot_h, c->blk_h, c->sc_h, c->x, H);
        quantize_row(c, c->x, H);
    }
    pthread_barrier_wait(&c->bar);
    if (c->head) project_share(c, t, c->head, c->head_s, H, g->vocab, c->logits);
    pthread_barrier_wait(&c->bar);
    return 0;
}

/* One decode step at position pos (the K/V cache holds rows 0..pos-1):
 * h [hidden] is the embedded token on entry and the residual on return;
 * logits [vocab]. head may be NULL (no head product). */
void orc_lm_step_i8(const orc_lm_geom *g, const orc_lm_layer_i8 *layers, float *kc, float *vc, int pos,
                    const float *cosv, const float *sinv, const float *final_norm, const int8_t *head,
                    const float *head_s, float *h, float *logits, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    const int64_t H = g->hidden, qd = g->heads * g->head_dim, kvd = g->kv_heads * g->head_dim, I = g->inter;
    const int64_t big = H > qd ? (H > 2 * I ? H : 2 * I) : (qd > 2 * I ? qd : 2 * I);
    lm_step_ctx c;
    memset(&c, 0, sizeof c);
    c.g = g, c.L = layers, c.kc = kc, c.vc = vc, c.cosv = cosv, c.sinv = sinv, c.final_norm = final_norm;
    c.head = head, c.head_s = head_s, c.h = h, c.logits = logits, c.pos = pos, c.threads = threads;
    float *mem = (float *)calloc((size_t)(big * 3 + qd + 2 * kvd + qd + (int64_t)threads * g->cap), sizeof(float));
    c.x = mem;
    c.tmp = c.x + big;
    c.act = c.tmp + big;
    c.qkv = c.act + big;
    c.ctx = c.qkv + qd + 2 * kvd;
    c.scores = c.ctx + qd;
    c.qa = (int8_t *)malloc((size_t)big);
    c.rot_h = (float *)malloc((size_t)(H + qd + I) * sizeof(float));
    c.rot_c = c.rot_h + H;
    c.rot_i = c.rot_c + qd;
    c.blk_h = orc_rotation(H, c.rot_h, &c.sc_h);
    c.blk_c = orc_rotation(qd, c.rot_c, &c.sc_c);
    c.blk_i = orc_rotation(I, c.rot_i, &c.sc_i);
    pthread_barrier_init(&c.bar, 0, (unsigned)threads);
    pthread_t tid[64];
    lm_worker w[64];
    for (int t = 0; t < threads; t++) {
        w[t] = (lm_worker){&c, t};
        if (t) pthread_create(&tid[t], 0, lm_step_worker, &w[t]);
    }
    lm_step_worker(&w[0]);
    for (int t = 1; t < threads; t++) pthread_join(tid[t], 0);
    pthread_barrier_destroy(&c.bar);
    free(c.qa);
    free(c.rot_h);
    free(mem);
}
