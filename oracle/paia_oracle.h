/* paia_oracle.h -- CPU oracle for the PAIA GEMV family (TEST INFRASTRUCTURE ONLY).
 *
 * This is a plain-C restatement of the reference's formats and GEMV semantics. It exists so that tests, the smoke
 * check and the benchmark's cpu_baseline leg can check the HIP library. The shipped product (libpaia_gemv.so, the
 * paia_gemv Python package, the torch ops) never links, imports or calls it.
 *
 * Every function names the reference file:line whose behaviour it restates. Paths are relative to the reference
 * repository root (Bejaine/PAIA-Project).
 *
 * Formats:
 *   e4m3fn     bias 7, no infinities, S.1111.111 is NaN, max finite 448     (src/paia_gemv/quant_host.h:1-5,18-23)
 *   fp16       IEEE binary16, RNE, subnormals, overflow to inf             (src/paia_gemv/quant_host.h:42-71)
 *   bf16       upper half of binary32, RNE                                 (src/tests/emulate_formats.py:26-28)
 *   INT4 ref   nibble n in 1..15, zero point 8, fp16 scale per 128 along K  (src/paia_gemv/quant_host.h:5-9,88-111)
 *   INT4 zp    nibble q in 0..15, 4-bit zero z per group, bf16 scale        (no reference code)
 *              zeros stored [N][ceil(G/2)] bytes, group 2j in the low nibble of byte j, 2j+1 in the high nibble.
 */
#ifndef PAIA_ORACLE_H
#define PAIA_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar formats ---- */
float po_e4m3_to_f32(uint8_t code);
uint8_t po_f32_to_e4m3(float v);
uint16_t po_f32_to_f16(float v);
float po_f16_to_f32(uint16_t h);
uint16_t po_f32_to_bf16(float v);
float po_bf16_to_f32(uint16_t b);

/* ---- quantizers (W is N x K row-major fp32) ---- */
void po_quantize_fp8_rowwise(const float* W, int N, int K, uint8_t* q, float* scale);
void po_quantize_int4_g128(const float* W, int N, int K, uint8_t* packed, uint16_t* scales_f16);
/* asymmetric INT4 (no reference code): min/max per group, bf16 scale, 4-bit zero point, (q - z) * s */
void po_quantize_int4_zp_g128(const float* W, int N, int K, uint8_t* packed, uint16_t* scales_bf16, uint8_t* zeros);

/* ---- dequantizers to fp32 [N][K] (bit-exact definitions) ---- */
void po_dequant_fp8(const uint8_t* q, const float* scale, int N, int K, float* out);
void po_dequant_int4(const uint8_t* packed, const uint16_t* scales_f16, int N, int K, float* out);
void po_dequant_int4_zp(const uint8_t* packed, const uint16_t* scales_bf16, const uint8_t* zeros, int N, int K,
                        float* out);
/* bf16 copy of the reference-format INT4 weights (what the unfused control materialises) */
void po_dequant_int4_bf16(const uint8_t* packed, const uint16_t* scales_f16, int N, int K, uint16_t* out_bf16);

/* ---- GEMV references: y[n] = sum_k Wd[n][k] * x[k] (+ bias[n]) ----
 * Wd is an fp32 [N][K] matrix (already dequantised); x and bias are bf16 bit patterns (bias may be NULL).
 * rows: optional list of nrows row indices (NULL = all N rows, nrows ignored); y gets one value per listed row. */
void po_gemv_f64(const float* Wd, const uint16_t* x_bf16, const uint16_t* bias_bf16, int N, int K,
                 const int* rows, int nrows, double* y);
void po_gemv_f32(const float* Wd, const uint16_t* x_bf16, const uint16_t* bias_bf16, int N, int K,
                 const int* rows, int nrows, float* y);

/* Fused per-row references straight from the quantised formats (no N x K fp32 buffer), fp64 accumulation. */
void po_gemv_fp8_f64(const uint8_t* q, const float* scale, const uint16_t* x_bf16, const uint16_t* bias_bf16,
                     int N, int K, const int* rows, int nrows, double* y);
void po_gemv_int4_f64(const uint8_t* packed, const uint16_t* scales_f16, const uint16_t* x_bf16, int N, int K,
                      const int* rows, int nrows, double* y);
void po_gemv_int4_zp_f64(const uint8_t* packed, const uint16_t* scales_bf16, const uint8_t* zeros,
                         const uint16_t* x_bf16, const uint16_t* bias_bf16, int N, int K, const int* rows, int nrows,
                         double* y);
void po_gemv_bf16_f64(const uint16_t* W_bf16, const uint16_t* x_bf16, const uint16_t* bias_bf16, int N, int K,
                      const int* rows, int nrows, double* y);

#ifdef __cplusplus
}
#endif
#endif
