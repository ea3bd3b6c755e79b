// On-device weight quantizers: the formats of src/paia_gemv/quant.py:8-31 and quant_host.h:74-106, produced on the
// GPU in one pass over W (fp32 [N][K], row-major). No reference C symbol: the reference quantizes with torch on the
// GPU; these are the same values from hand-written gfx950 kernels.
//
//   FP8 rowwise  scale[n] = amax_n / 448 (1 if the row is all zero); q = e4m3_rn(clamp(w / scale, +-448)).
//                One workgroup per row: amax by wave DPP max + LDS, then the row is re-read (from L2) and encoded
//                four values per lane with the gfx950 OCP e4m3 convert (round to nearest even).
//   INT4 g128    s16 = f16_rn(amax_g / 7) (1 if the group is all zero); sf = float(s16) (1 if it underflowed to 0);
//                n = clamp(rint(w / sf), -7, 7) + 8, packed two per byte (weight 2j low nibble).
//                One wave per group of 128: two values per lane, one packed byte per lane.
//   INT4 g128 asymmetric (no reference counterpart; the format of the BASELINE INT4 configs, dequant (q - z) * s):
//                lo = min(0, min w), hi = max(0, max w) over the group; s = bf16_rn((hi - lo) / 15) (1 if that is 0);
//                z = clamp(rint(-lo / s), 0, 15); q = clamp(rint(w / s) + z, 0, 15). Zero points are packed two
//                groups per byte along G, so one wave handles a pair of groups.
// Divisions are IEEE (correctly rounded), rint rounds half to even, as torch.round and std::nearbyint do.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_kernel.h"
#include "paia_gemv.h"

namespace paia {

__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x124>(v));
    v = fmaxf(v, dpp_f32<0x128>(v));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}
__device__ __forceinline__ float wave_min(float v) { return -wave_max(-v); }

// four fp32 -> four e4m3 codes (byte i = value i), round to nearest even; |v| <= 448 on entry
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d)
{
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return (uint32_t)w;
}

constexpr int kQBlock = 256;

__global__ void __launch_bounds__(kQBlock) quantize_fp8_kernel(const float* __restrict__ W, uint8_t* __restrict__ q,
                                                               float* __restrict__ scale, int N, int K)
{
    __shared__ float red[kQBlock / kWave];
    const int K4 = K / 4;
    for (int n = (int)blockIdx.x; n < N; n += (int)gridDim.x) {
        const float4* row = reinterpret_cast<const float4*>(W + (size_t)n * K);
        float amax = 0.0f;
        for (int i = (int)threadIdx.x; i < K4; i += kQBlock) {
            const float4 v = row[i];
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        amax = wave_max(amax);
        if (lane_id() == 0) red[wave_id()] = amax;
        __syncthreads();
        amax = red[0];
#pragma unroll
        for (int w = 1; w < kQBlock / kWave; ++w) amax = fmaxf(amax, red[w]);
        __syncthreads();                                   // red is reused by the next row
        const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
        if (threadIdx.x == 0) scale[n] = s;
        uint32_t* qrow = reinterpret_cast<uint32_t*>(q + (size_t)n * K);
        for (int i = (int)threadIdx.x; i < K4; i += kQBlock) {
            const float4 v = row[i];
            const float a = fminf(fmaxf(v.x / s, -448.0f), 448.0f), b = fminf(fmaxf(v.y / s, -448.0f), 448.0f);
            const float c = fminf(fmaxf(v.z / s, -448.0f), 448.0f), d = fminf(fmaxf(v.w / s, -448.0f), 448.0f);
            qrow[i] = e4m3x4(a, b, c, d);
        }
    }
}

// One wave per group of 128 (4 groups per 256-thread block, grid-stride over N*G groups).
__global__ void __launch_bounds__(kQBlock) quantize_int4_kernel(const float* __restrict__ W,
                                                                uint8_t* __restrict__ packed,
                                                                uint16_t* __restrict__ scales, int N, int K)
{
    const int G = K / 128;
    const size_t ngroups = (size_t)N * (size_t)G;
    const int lane = lane_id();
    for (size_t gi = (size_t)blockIdx.x * (kQBlock / kWave) + (size_t)wave_id(); gi < ngroups;
         gi += (size_t)gridDim.x * (kQBlock / kWave)) {
        const size_t n = gi / (size_t)G, g = gi - n * (size_t)G;
        const float2 v = reinterpret_cast<const float2*>(W + n * (size_t)K + g * 128)[lane];
        const float amax = wave_max(fmaxf(fabsf(v.x), fabsf(v.y)));
        const _Float16 s16 = (_Float16)(amax > 0.0f ? amax / 7.0f : 1.0f);   // v_cvt_f16_f32: round to nearest even
        float sf = (float)s16;
        if (!(sf > 0.0f)) sf = 1.0f;
        const int q0 = (int)fminf(fmaxf(__builtin_rintf(v.x / sf), -7.0f), 7.0f) + 8;
        const int q1 = (int)fminf(fmaxf(__builtin_rintf(v.y / sf), -7.0f), 7.0f) + 8;
        packed[n * (size_t)(K / 2) + g * 64 + (size_t)lane] = (uint8_t)(q0 | (q1 << 4));
        if (lane == 0) scales[gi] = __builtin_bit_cast(uint16_t, s16);
    }
}

// One wave per pair of groups (2j, 2j+1) of a row, so the packed zero-point byte has one writer.
__global__ void __launch_bounds__(kQBlock) quantize_int4_zp_kernel(const float* __restrict__ W,
                                                                   uint8_t* __restrict__ packed,
                                                                   uint16_t* __restrict__ scales,
                                                                   uint8_t* __restrict__ zeros, int N, int K)
{
    const int G = K / 128, ZB = (G + 1) / 2;
    const size_t npairs = (size_t)N * (size_t)ZB;
    const int lane = lane_id();
    for (size_t pi = (size_t)blockIdx.x * (kQBlock / kWave) + (size_t)wave_id(); pi < npairs;
         pi += (size_t)gridDim.x * (kQBlock / kWave)) {
        const size_t n = pi / (size_t)ZB, j = pi - n * (size_t)ZB;
        uint32_t zbyte = 0;
        for (int h = 0; h < 2; ++h) {
            const size_t g = 2 * j + (size_t)h;
            if (g >= (size_t)G) break;                     // odd G: the last byte has one group (high nibble 0)
            const float2 v = reinterpret_cast<const float2*>(W + n * (size_t)K + g * 128)[lane];
            const float lo = fminf(wave_min(fminf(v.x, v.y)), 0.0f);
            const float hi = fmaxf(wave_max(fmaxf(v.x, v.y)), 0.0f);
            const float r = (hi - lo) / 15.0f;
            uint32_t sb = f32_to_bf16_rne(r);
            float s = bf16_to_f32(sb);
            if (!(s > 0.0f)) {
                sb = 0x3F80u;                              // bf16 1.0
                s = 1.0f;
            }
            const float zf = fminf(fmaxf(__builtin_rintf(-lo / s), 0.0f), 15.0f);
            const int q0 = (int)fminf(fmaxf(__builtin_rintf(v.x / s) + zf, 0.0f), 15.0f);
            const int q1 = (int)fminf(fmaxf(__builtin_rintf(v.y / s) + zf, 0.0f), 15.0f);
            packed[n * (size_t)(K / 2) + g * 64 + (size_t)lane] = (uint8_t)(q0 | (q1 << 4));
            if (lane == 0) scales[n * (size_t)G + g] = (uint16_t)sb;
            zbyte |= (uint32_t)zf << (4 * h);
        }
        if (lane == 0) zeros[pi] = (uint8_t)zbyte;
    }
}

}  // namespace paia

namespace {
using namespace paia;

unsigned qgrid(size_t units, size_t per_block)
{
    const size_t want = (units + per_block - 1) / per_block;
    return (unsigned)(want < 16384 ? (want > 0 ? want : 1) : 16384);
}

}  // namespace

extern "C" {

int paia_quantize_fp8_rowwise(const void* W, void* q, void* scale, int N, int K, void* stream)
{
    if (N <= 0 || K <= 0 || (K & 15) || !aligned(W, 16) || !aligned(q, 16) || !aligned(scale, 4)) return -2;
    hipLaunchKernelGGL(quantize_fp8_kernel, dim3(qgrid((size_t)N, 1)), dim3(kQBlock), 0,
                       static_cast<hipStream_t>(stream), static_cast<const float*>(W), static_cast<uint8_t*>(q),
                       static_cast<float*>(scale), N, K);
    return (int)hipGetLastError();
}

int paia_quantize_int4_g128(const void* W, void* packed, void* scales, int N, int K, void* stream)
{
    if (N <= 0 || K <= 0 || (K & 127) || !aligned(W, 16) || !aligned(packed, 16) || !aligned(scales, 2)) return -2;
    hipLaunchKernelGGL(quantize_int4_kernel, dim3(qgrid((size_t)N * (size_t)(K / 128), kQBlock / kWave)),
                       dim3(kQBlock), 0, static_cast<hipStream_t>(stream), static_cast<const float*>(W),
                       static_cast<uint8_t*>(packed), static_cast<uint16_t*>(scales), N, K);
    return (int)hipGetLastError();
}

int paia_quantize_int4_zp_g128(const void* W, void* packed, void* scales, void* zeros, int N, int K, void* stream)
{
    if (N <= 0 || K <= 0 || (K & 127) || !aligned(W, 16) || !aligned(packed, 16) || !aligned(scales, 2) ||
        zeros == nullptr)
        return -2;
    const size_t pairs = (size_t)N * (size_t)((K / 128 + 1) / 2);
    hipLaunchKernelGGL(quantize_int4_zp_kernel, dim3(qgrid(pairs, kQBlock / kWave)), dim3(kQBlock), 0,
                       static_cast<hipStream_t>(stream), static_cast<const float*>(W), static_cast<uint8_t*>(packed),
                       static_cast<uint16_t*>(scales), static_cast<uint8_t*>(zeros), N, K);
    return (int)hipGetLastError();
}

}  // extern "C"
