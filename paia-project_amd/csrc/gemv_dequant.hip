// Dequantisation to fp32 [N][K] -- the bit-exact definitions the fused kernels compute in registers.
// No reference C symbol: the reference dequantises with torch (src/paia_gemv/quant.py:16-17,34-38) and on the host
// (quant_host.h:82-85,106-111). These kernels give the same values on the GPU:
//   FP8      out = float(e4m3(q)) * scale[n]            one fp32 product (round to nearest even)
//   INT4     out = (n - 8) * float(s_fp16)              exact in fp32
//   INT4ZP   out = (q - z) * float(s_bf16)              exact in fp32
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_kernel.h"
#include "paia_gemv.h"

namespace paia {

// 16 e4m3 weights per thread-iteration -> 64 bytes of fp32.
__global__ void __launch_bounds__(256) dequant_fp8_kernel(const uint8_t* __restrict__ Wq,
                                                          const float* __restrict__ scale, float* __restrict__ out,
                                                          size_t units, int K)
{
    const size_t per_row = (size_t)K / 16;
    for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += (size_t)gridDim.x * blockDim.x) {
        const size_t row = u / per_row;
        const float s = scale[row];
        const u32x4 w = *reinterpret_cast<const u32x4*>(Wq + u * 16);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
        float4* o = reinterpret_cast<float4*>(out + u * 16);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(ws[j], false);
            const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(ws[j], true);
            o[j] = make_float4(lo[0] * s, lo[1] * s, hi[0] * s, hi[1] * s);
        }
    }
}

// 32 nibbles per thread-iteration -> 128 bytes of fp32. ZP: asymmetric format (bf16 scale, 4-bit zero), else the
// reference format (fp16 scale, zero 8).
template <bool ZP>
__global__ void __launch_bounds__(256) dequant_int4_kernel(const uint8_t* __restrict__ Wq,
                                                           const uint16_t* __restrict__ scales,
                                                           const uint8_t* __restrict__ zeros, float* __restrict__ out,
                                                           size_t units, int K)
{
    const size_t per_row = (size_t)K / 32;
    const int G = K / 128, ZB = (G + 1) / 2;
    for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += (size_t)gridDim.x * blockDim.x) {
        const size_t row = u / per_row;
        const int k0 = (int)(u - row * per_row) * 32;
        const int g = k0 >> 7;
        float s, z;
        if constexpr (ZP) {
            s = bf16_to_f32(scales[row * (size_t)G + (size_t)g]);
            z = (float)((zeros[row * (size_t)ZB + (size_t)(g >> 1)] >> ((g & 1) * 4)) & 0xFu);
        } else {
            s = f16_to_f32(scales[row * (size_t)G + (size_t)g]);
            z = 8.0f;
        }
        const u32x4 w = *reinterpret_cast<const u32x4*>(Wq + u * 16);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
        float4* o = reinterpret_cast<float4*>(out + u * 32);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float v[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) v[t] = ((float)((ws[j] >> (4 * t)) & 0xFu) - z) * s;
            o[2 * j] = make_float4(v[0], v[1], v[2], v[3]);
            o[2 * j + 1] = make_float4(v[4], v[5], v[6], v[7]);
        }
    }
}

}  // namespace paia

namespace {
using namespace paia;

unsigned grid_for(size_t units)
{
    const size_t want = (units + 255) / 256;
    return (unsigned)(want < 16384 ? want : 16384);
}

}  // namespace

extern "C" {

// Wq [N][K] e4m3 bytes, scale [N] fp32 -> out [N][K] fp32. K % 16 == 0; Wq, out 16 B aligned; scale 4 B aligned.
int paia_dequant_fp8(const void* Wq, const void* scale, void* out, int N, int K, void* stream)
{
    if (N <= 0 || K <= 0 || (K & 15) || !aligned(Wq, 16) || !aligned(out, 16) || !aligned(scale, 4)) return -2;
    const size_t units = (size_t)N * (size_t)K / 16;
    hipLaunchKernelGGL(dequant_fp8_kernel, dim3(grid_for(units)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint8_t*>(Wq), static_cast<const float*>(scale), static_cast<float*>(out),
                       units, K);
    return (int)hipGetLastError();
}

// Reference INT4: Wq [N][K/2], scales fp16 [N][K/128] -> out [N][K] fp32. K % 128 == 0.
int paia_dequant_int4(const void* Wq, const void* scales, void* out, int N, int K, void* stream)
{
    if (N <= 0 || K <= 0 || (K & 127) || !aligned(Wq, 16) || !aligned(out, 16) || !aligned(scales, 2)) return -2;
    const size_t units = (size_t)N * (size_t)K / 32;
    hipLaunchKernelGGL(dequant_int4_kernel<false>, dim3(grid_for(units)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(Wq),
                       static_cast<const uint16_t*>(scales), static_cast<const uint8_t*>(nullptr),
                       static_cast<float*>(out), units, K);
    return (int)hipGetLastError();
}

// Asymmetric INT4: Wq [N][K/2], scales bf16 [N][G], zeros [N][ceil(G/2)] -> out [N][K] fp32. K % 128 == 0.
int paia_dequant_int4_zp(const void* Wq, const void* scales, const void* zeros, void* out, int N, int K, void* stream)
{
    if (N <= 0 || K <= 0 || (K & 127) || !aligned(Wq, 16) || !aligned(out, 16) || !aligned(scales, 2) ||
        zeros == nullptr)
        return -2;
    const size_t units = (size_t)N * (size_t)K / 32;
    hipLaunchKernelGGL(dequant_int4_kernel<true>, dim3(grid_for(units)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(Wq),
                       static_cast<const uint16_t*>(scales), static_cast<const uint8_t*>(zeros),
                       static_cast<float*>(out), units, K);
    return (int)hipGetLastError();
}

}  // extern "C"
