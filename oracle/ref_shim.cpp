// ref_shim.cpp -- TEST INFRASTRUCTURE. Exposes the reference's own host-format functions with C linkage so the tests
// can compare the oracle restatement against the reference implementation itself.
//
// It includes src/paia_gemv/quant_host.h from the reference checkout (passed with -I by oracle/Makefile); nothing of
// the reference is copied here. The build output goes to oracle/_ref/ (git-ignored) and exists only where the
// reference checkout was present at build time.
#include <cstdint>

#include "quant_host.h"

extern "C" {

float ref_e4m3_decode(uint8_t b) { return paia_host::e4m3_decode(b); }
uint8_t ref_e4m3_encode(float x) { return paia_host::e4m3_encode(x); }
uint16_t ref_f32_to_f16_bits(float f) { return paia_host::f32_to_f16_bits(f); }
float ref_f16_bits_to_f32(uint16_t h) { return paia_host::f16_bits_to_f32(h); }

void ref_quantize_fp8_rowwise(const float* W, int N, int K, uint8_t* q, float* scale)
{
    paia_host::quantize_fp8_rowwise(W, N, K, q, scale);
}

void ref_dequant_fp8(const uint8_t* q, const float* scale, int N, int K, float* out)
{
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k) out[(size_t)n * K + k] = paia_host::dequant_fp8(q, scale, K, n, k);
}

void ref_quantize_int4_g128(const float* W, int N, int K, uint8_t* packed, uint16_t* scales)
{
    paia_host::quantize_int4_g128(W, N, K, packed, scales);
}

void ref_dequant_int4(const uint8_t* packed, const uint16_t* scales, int N, int K, float* out)
{
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k) out[(size_t)n * K + k] = paia_host::dequant_int4(packed, scales, K, n, k);
}

}  // extern "C"
