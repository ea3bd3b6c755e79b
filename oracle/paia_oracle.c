/* paia_oracle.c -- CPU oracle for the PAIA GEMV family. TEST INFRASTRUCTURE ONLY: only tests/, the smoke check and
 * bench.py's cpu_baseline leg may load it, and only as the checker. The product never calls it.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, so every fp32 product/sum below is one IEEE-rounded operation).
 * The conversions are written arithmetically (frexp/rint on exactly-scaled values) rather than as bit tricks; they
 * realise the same rounding rules as the reference's definitions cited at each function.
 */
#include "paia_oracle.h"

#include <math.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------------------------- */
/* e4m3fn                                                                                                          */
/* ------------------------------------------------------------------------------------------------------------- */

/* Follows src/paia_gemv/quant_host.h:18-23 (and src/tests/emulate_formats.py:35-41): value = (-1)^s * 2^(e-7) *
 * (1 + m/8) for e > 0, 2^-6 * m/8 for e == 0; S.1111.111 is NaN (returned unsigned, as the reference does). */
float po_e4m3_to_f32(uint8_t code)
{
    const unsigned ex = (code >> 3) & 0xFu, man = code & 0x7u;
    if (ex == 0xFu && man == 0x7u) return NAN;
    /* (8 + m) * 2^(e - 10) == (1 + m/8) * 2^(e - 7);  m * 2^-9 == 2^-6 * m/8 */
    const float mag = ex ? ldexpf((float)(8u + man), (int)ex - 10) : ldexpf((float)man, -9);
    return (code & 0x80u) ? -mag : mag;
}

/* Follows src/paia_gemv/quant_host.h:25-39: nearest code, ties to the even code, |v| clamped to 448 first.
 * (The reference finds the nearest code by a table search; it is the RNE of the 3-bit mantissa, done here with rintf
 * on exactly scaled values.) A NaN input maps to a signed zero, which is what the reference's table search yields
 * (its comparisons with NaN are all false, so it keeps code 0). */
uint8_t po_f32_to_e4m3(float v)
{
    const uint8_t sign = signbit(v) ? 0x80u : 0u;
    float a = fabsf(v);
    if (isnan(a)) return sign;
    if (a > 448.0f) a = 448.0f;
    if (a < 0.015625f) {                       /* below 2^-6: uniform grid of 2^-9, codes 0..8 (8 is 2^-6) */
        return (uint8_t)(sign | (uint8_t)rintf(a * 512.0f));
    }
    int e2;
    const float fr = frexpf(a, &e2);           /* a = fr * 2^e2, fr in [0.5, 1) */
    int ub = e2 - 1;                           /* a = (1 + f) * 2^ub, f = 2 fr - 1 */
    int m = (int)rintf((2.0f * fr - 1.0f) * 8.0f);
    if (m == 8) { m = 0; ++ub; }               /* mantissa carry into the exponent */
    return (uint8_t)(sign | (uint8_t)(((ub + 7) << 3) | m));
}

/* ------------------------------------------------------------------------------------------------------------- */
/* fp16, bf16                                                                                                      */
/* ------------------------------------------------------------------------------------------------------------- */

/* Follows src/paia_gemv/quant_host.h:41-61: IEEE binary16 round-to-nearest-even, subnormals, overflow to inf,
 * NaN -> quiet NaN 0x7E00 (with sign). Computed in double on exactly scaled values. */
uint16_t po_f32_to_f16(float v)
{
    const uint16_t sign = signbit(v) ? 0x8000u : 0u;
    if (isnan(v)) return (uint16_t)(sign | 0x7E00u);
    const double a = fabs((double)v);
    if (isinf(a)) return (uint16_t)(sign | 0x7C00u);
    if (a < 6.103515625e-05) {                 /* below 2^-14: subnormal grid of 2^-24, code 0x400 = 2^-14 */
        return (uint16_t)(sign | (uint16_t)rint(a * 16777216.0));
    }
    int e2;
    const double fr = frexp(a, &e2);
    int ub = e2 - 1;
    int m = (int)rint((2.0 * fr - 1.0) * 1024.0);
    if (m == 1024) { m = 0; ++ub; }
    if (ub > 15) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | (uint16_t)(((ub + 15) << 10) | m));
}

/* Follows src/paia_gemv/quant_host.h:63-71. */
float po_f16_to_f32(uint16_t h)
{
    const unsigned ex = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    float mag;
    if (ex == 0x1Fu) mag = man ? NAN : INFINITY;
    else if (ex == 0u) mag = ldexpf((float)man, -24);
    else mag = ldexpf((float)(1024u + man), (int)ex - 25);
    return (h & 0x8000u) ? -mag : mag;
}

/* Follows src/tests/emulate_formats.py:26-28 (round to nearest even on the upper 16 bits); NaN stays a quiet NaN. */
uint16_t po_f32_to_bf16(float v)
{
    uint32_t u;
    memcpy(&u, &v, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    const uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7FFFu + lsb) >> 16);
}

float po_bf16_to_f32(uint16_t b)
{
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ------------------------------------------------------------------------------------------------------------- */
/* quantizers                                                                                                      */
/* ------------------------------------------------------------------------------------------------------------- */

/* Follows src/paia_gemv/quant_host.h:73-81 and src/paia_gemv/quant.py:8-13: scale = amax/448 (1 if amax == 0),
 * q = e4m3_rn(W / scale) with the +-448 clamp. */
void po_quantize_fp8_rowwise(const float* W, int N, int K, uint8_t* q, float* scale)
{
    for (int n = 0; n < N; ++n) {
        const float* w = W + (size_t)n * (size_t)K;
        float amax = 0.0f;
        for (int k = 0; k < K; ++k) {
            const float a = fabsf(w[k]);
            if (a > amax) amax = a;
        }
        const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
        scale[n] = s;
        uint8_t* qr = q + (size_t)n * (size_t)K;
        for (int k = 0; k < K; ++k) qr[k] = po_f32_to_e4m3(w[k] / s);
    }
}

/* Follows src/paia_gemv/quant_host.h:87-105 and src/paia_gemv/quant.py:20-31: per group of 128 along K,
 * s16 = fp16(amax/7) (amax == 0 -> 1.0); quantise with sf = float(s16), or 1.0 when sf underflowed to 0;
 * n = clamp(rint(w/sf), -7, 7) + 8; byte j of a row holds weight 2j (low nibble) and 2j+1 (high nibble). */
void po_quantize_int4_g128(const float* W, int N, int K, uint8_t* packed, uint16_t* scales_f16)
{
    const int G = K / 128;
    for (int n = 0; n < N; ++n) {
        for (int g = 0; g < G; ++g) {
            const float* w = W + (size_t)n * (size_t)K + (size_t)g * 128u;
            float amax = 0.0f;
            for (int i = 0; i < 128; ++i) {
                const float a = fabsf(w[i]);
                if (a > amax) amax = a;
            }
            const uint16_t s16 = po_f32_to_f16(amax > 0.0f ? amax / 7.0f : 1.0f);
            scales_f16[(size_t)n * (size_t)G + (size_t)g] = s16;
            float sf = po_f16_to_f32(s16);
            if (!(sf > 0.0f)) sf = 1.0f;
            uint8_t* dst = packed + (size_t)n * (size_t)(K / 2) + (size_t)g * 64u;
            for (int i = 0; i < 64; ++i) {
                int lo = (int)rintf(w[2 * i] / sf), hi = (int)rintf(w[2 * i + 1] / sf);
                lo = (lo < -7 ? -7 : (lo > 7 ? 7 : lo)) + 8;
                hi = (hi < -7 ? -7 : (hi > 7 ? 7 : hi)) + 8;
                dst[i] = (uint8_t)(lo | (hi << 4));
            }
        }
    }
}

/* Asymmetric INT4 g128 (no reference code; the format of the BASELINE INT4 configs, dequant (q - z) * s): per group,
 * lo = min(0, min w), hi = max(0, max w), s = bf16_rn((hi - lo) / 15) (bf16 1.0 if that is 0),
 * z = clamp(rint(-lo / s), 0, 15), q = clamp(rint(w / s) + z, 0, 15). zeros [N][ceil(G/2)], group 2j low nibble. */
void po_quantize_int4_zp_g128(const float* W, int N, int K, uint8_t* packed, uint16_t* scales_bf16, uint8_t* zeros)
{
    const int G = K / 128, ZB = (G + 1) / 2;
    for (int n = 0; n < N; ++n) {
        for (int j = 0; j < ZB; ++j) zeros[(size_t)n * (size_t)ZB + (size_t)j] = 0;
        for (int g = 0; g < G; ++g) {
            const float* w = W + (size_t)n * (size_t)K + (size_t)g * 128u;
            float lo = 0.0f, hi = 0.0f;
            for (int i = 0; i < 128; ++i) {
                if (w[i] < lo) lo = w[i];
                if (w[i] > hi) hi = w[i];
            }
            uint16_t sb = po_f32_to_bf16((hi - lo) / 15.0f);
            float s = po_bf16_to_f32(sb);
            if (!(s > 0.0f)) {
                sb = 0x3F80u;
                s = 1.0f;
            }
            float zf = rintf(-lo / s);
            zf = zf < 0.0f ? 0.0f : (zf > 15.0f ? 15.0f : zf);
            scales_bf16[(size_t)n * (size_t)G + (size_t)g] = sb;
            zeros[(size_t)n * (size_t)ZB + (size_t)(g >> 1)] |= (uint8_t)((unsigned)zf << ((g & 1) * 4));
            uint8_t* dst = packed + (size_t)n * (size_t)(K / 2) + (size_t)g * 64u;
            for (int i = 0; i < 64; ++i) {
                float a = rintf(w[2 * i] / s) + zf, b = rintf(w[2 * i + 1] / s) + zf;
                a = a < 0.0f ? 0.0f : (a > 15.0f ? 15.0f : a);
                b = b < 0.0f ? 0.0f : (b > 15.0f ? 15.0f : b);
                dst[i] = (uint8_t)((unsigned)a | ((unsigned)b << 4));
            }
        }
    }
}

/* ------------------------------------------------------------------------------------------------------------- */
/* dequantizers                                                                                                    */
/* ------------------------------------------------------------------------------------------------------------- */

static inline unsigned nibble_at(const uint8_t* row, int k) { return (row[k >> 1] >> ((k & 1) * 4)) & 0xFu; }

/* Follows src/paia_gemv/quant.py:16-17 and quant_host.h:82-85: float(e4m3) * scale[n], one fp32 product.
 * (The 256 code values are taken from po_e4m3_to_f32 once.) */
void po_dequant_fp8(const uint8_t* q, const float* scale, int N, int K, float* out)
{
    float tab[256];
    for (int c = 0; c < 256; ++c) tab[c] = po_e4m3_to_f32((uint8_t)c);
    for (int n = 0; n < N; ++n) {
        const uint8_t* qr = q + (size_t)n * (size_t)K;
        float* o = out + (size_t)n * (size_t)K;
        const float s = scale[n];
        for (int k = 0; k < K; ++k) o[k] = tab[qr[k]] * s;
    }
}

/* Follows src/paia_gemv/quant.py:34-38 and quant_host.h:106-111: (n - 8) * float(s16) (exact in fp32). */
void po_dequant_int4(const uint8_t* packed, const uint16_t* scales_f16, int N, int K, float* out)
{
    const int G = K / 128;
    for (int n = 0; n < N; ++n) {
        const uint8_t* row = packed + (size_t)n * (size_t)(K / 2);
        for (int k = 0; k < K; ++k)
            out[(size_t)n * K + k] = (float)((int)nibble_at(row, k) - 8) * po_f16_to_f32(scales_f16[(size_t)n * G + k / 128]);
    }
}

/* No reference code: (q - z) * float(s_bf16), exact in fp32 (5-bit integer x 8-bit
 * significand). zeros: [N][ceil(G/2)] bytes, group g in nibble (g & 1) of byte g/2. */
void po_dequant_int4_zp(const uint8_t* packed, const uint16_t* scales_bf16, const uint8_t* zeros, int N, int K,
                        float* out)
{
    const int G = K / 128, ZB = (G + 1) / 2;
    for (int n = 0; n < N; ++n) {
        const uint8_t* row = packed + (size_t)n * (size_t)(K / 2);
        const uint8_t* zr = zeros + (size_t)n * (size_t)ZB;
        for (int k = 0; k < K; ++k) {
            const int g = k / 128;
            const int z = (int)((zr[g >> 1] >> ((g & 1) * 4)) & 0xFu);
            out[(size_t)n * K + k] = (float)((int)nibble_at(row, k) - z) * po_bf16_to_f32(scales_bf16[(size_t)n * G + g]);
        }
    }
}

/* Follows src/paia_gemv/gemv_int4.cuh:155-174 (the unfused control's first stage): bf16_rn((n - 8) * s). */
void po_dequant_int4_bf16(const uint8_t* packed, const uint16_t* scales_f16, int N, int K, uint16_t* out_bf16)
{
    const int G = K / 128;
    for (int n = 0; n < N; ++n) {
        const uint8_t* row = packed + (size_t)n * (size_t)(K / 2);
        for (int k = 0; k < K; ++k) {
            const float v = (float)((int)nibble_at(row, k) - 8) * po_f16_to_f32(scales_f16[(size_t)n * G + k / 128]);
            out_bf16[(size_t)n * K + k] = po_f32_to_bf16(v);
        }
    }
}

/* ------------------------------------------------------------------------------------------------------------- */
/* GEMV references                                                                                                 */
/* ------------------------------------------------------------------------------------------------------------- */

static inline int row_of(const int* rows, int i) { return rows ? rows[i] : i; }
static inline double bias_of(const uint16_t* bias, int n) { return bias ? (double)po_bf16_to_f32(bias[n]) : 0.0; }

/* fp64 dot of a dequantised row with x: the reference's own check method (src/tests/gemv_bf16_check.cu:85-90,327). */
void po_gemv_f64(const float* Wd, const uint16_t* x_bf16, const uint16_t* bias_bf16, int N, int K, const int* rows,
                 int nrows, double* y)
{
    const int cnt = rows ? nrows : N;
    for (int i = 0; i < cnt; ++i) {
        const int n = row_of(rows, i);
        const float* w = Wd + (size_t)n * (size_t)K;
        double s = 0.0;
        for (int k = 0; k < K; ++k) s += (double)w[k] * (double)po_bf16_to_f32(x_bf16[k]);
        y[i] = s + bias_of(bias_bf16, n);
    }
}

/* fp32 sequential accumulation (an fp32-accumulated reference; one rounding per product and per sum). */
void po_gemv_f32(const float* Wd, const uint16_t* x_bf16, const uint16_t* bias_bf16, int N, int K, const int* rows,
                 int nrows, float* y)
{
    const int cnt = rows ? nrows : N;
    for (int i = 0; i < cnt; ++i) {
        const int n = row_of(rows, i);
        const float* w = Wd + (size_t)n * (size_t)K;
        float s = 0.0f;
        for (int k = 0; k < K; ++k) {
            const float p = w[k] * po_bf16_to_f32(x_bf16[k]);
            s = s + p;
        }
        y[i] = s + (bias_bf16 ? po_bf16_to_f32(bias_bf16[n]) : 0.0f);
    }
}

void po_gemv_bf16_f64(const uint16_t* W_bf16, const uint16_t* x_bf16, const uint16_t* bias_bf16, int N, int K,
                      const int* rows, int nrows, double* y)
{
    const int cnt = rows ? nrows : N;
    for (int i = 0; i < cnt; ++i) {
        const int n = row_of(rows, i);
        const uint16_t* w = W_bf16 + (size_t)n * (size_t)K;
        double s = 0.0;
        for (int k = 0; k < K; ++k) s += (double)po_bf16_to_f32(w[k]) * (double)po_bf16_to_f32(x_bf16[k]);
        y[i] = s + bias_of(bias_bf16, n);
    }
}

void po_gemv_fp8_f64(const uint8_t* q, const float* scale, const uint16_t* x_bf16, const uint16_t* bias_bf16, int N,
                     int K, const int* rows, int nrows, double* y)
{
    const int cnt = rows ? nrows : N;
    for (int i = 0; i < cnt; ++i) {
        const int n = row_of(rows, i);
        const uint8_t* qr = q + (size_t)n * (size_t)K;
        double s = 0.0;
        for (int k = 0; k < K; ++k)
            s += (double)(po_e4m3_to_f32(qr[k]) * scale[n]) * (double)po_bf16_to_f32(x_bf16[k]);
        y[i] = s + bias_of(bias_bf16, n);
    }
}

void po_gemv_int4_f64(const uint8_t* packed, const uint16_t* scales_f16, const uint16_t* x_bf16, int N, int K,
                      const int* rows, int nrows, double* y)
{
    const int cnt = rows ? nrows : N, G = K / 128;
    for (int i = 0; i < cnt; ++i) {
        const int n = row_of(rows, i);
        const uint8_t* row = packed + (size_t)n * (size_t)(K / 2);
        double s = 0.0;
        for (int k = 0; k < K; ++k) {
            const double w = (double)((int)nibble_at(row, k) - 8) * (double)po_f16_to_f32(scales_f16[(size_t)n * G + k / 128]);
            s += w * (double)po_bf16_to_f32(x_bf16[k]);
        }
        y[i] = s;
    }
}

void po_gemv_int4_zp_f64(const uint8_t* packed, const uint16_t* scales_bf16, const uint8_t* zeros,
                         const uint16_t* x_bf16, const uint16_t* bias_bf16, int N, int K, const int* rows, int nrows,
                         double* y)
{
    const int cnt = rows ? nrows : N, G = K / 128, ZB = (G + 1) / 2;
    for (int i = 0; i < cnt; ++i) {
        const int n = row_of(rows, i);
        const uint8_t* row = packed + (size_t)n * (size_t)(K / 2);
        const uint8_t* zr = zeros + (size_t)n * (size_t)ZB;
        double s = 0.0;
        for (int k = 0; k < K; ++k) {
            const int g = k / 128;
            const int z = (int)((zr[g >> 1] >> ((g & 1) * 4)) & 0xFu);
            const double w = (double)((int)nibble_at(row, k) - z) * (double)po_bf16_to_f32(scales_bf16[(size_t)n * G + g]);
            s += w * (double)po_bf16_to_f32(x_bf16[k]);
        }
        y[i] = s + bias_of(bias_bf16, n);
    }
}
