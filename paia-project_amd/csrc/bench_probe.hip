// Measurement kernels for the benchmark harness (libpaia_probe.so; not part of the GEMV library).
//
// paia_probe_read: a pure streaming read, 16-byte nontemporal loads with a grid-stride loop and an XOR sink that
//   keeps the loads alive -- the MI355X counterpart of the reference's dev read probe "B0"
//   (src/tests/gemv_bf16_check.cu:131-139,228-252). Timing it on the same byte counts as a GEMV gives the achievable
//   bandwidth (and the fixed cost) that kernel is measured against.
// paia_probe_copy: a plain 16-byte-per-lane copy of known size, the calibration kernel for the rocprofv3 byte counters
//   (FETCH_SIZE should read its size once, WRITE_SIZE its size once).
// paia_probe_empty: an empty kernel, for the per-launch floor of back-to-back launches in a graph.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int UNROLL>
__global__ void __launch_bounds__(256) read_probe_kernel(const u32x4* __restrict__ p, size_t n16, uint32_t* sink)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (UNROLL - 1) * stride < n16; i += UNROLL * stride) {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const u32x4 v = __builtin_nontemporal_load(p + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;   // practically never true; keeps the loads from being removed
}

__global__ void __launch_bounds__(256) copy_probe_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                         size_t n16)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

__global__ void empty_kernel() {}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) int paia_probe_read(const void* buf, size_t nbytes, void* sink, int grid,
                                                           int unroll, void* stream)
{
    if (!buf || !sink || (reinterpret_cast<uintptr_t>(buf) & 15) || grid <= 0) return -2;
    const size_t n16 = nbytes / 16;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const u32x4* p = static_cast<const u32x4*>(buf);
    uint32_t* s = static_cast<uint32_t*>(sink);
    switch (unroll) {
    case 1: hipLaunchKernelGGL(read_probe_kernel<1>, dim3(grid), dim3(256), 0, st, p, n16, s); break;
    case 4: hipLaunchKernelGGL(read_probe_kernel<4>, dim3(grid), dim3(256), 0, st, p, n16, s); break;
    case 8: hipLaunchKernelGGL(read_probe_kernel<8>, dim3(grid), dim3(256), 0, st, p, n16, s); break;
    default: return -1;
    }
    return (int)hipGetLastError();
}

__attribute__((visibility("default"))) int paia_probe_copy(const void* src, void* dst, size_t nbytes, int grid,
                                                           void* stream)
{
    if (!src || !dst || ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) || grid <= 0)
        return -2;
    hipLaunchKernelGGL(copy_probe_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), nbytes / 16);
    return (int)hipGetLastError();
}

__attribute__((visibility("default"))) int paia_probe_empty(int grid, void* stream)
{
    hipLaunchKernelGGL(empty_kernel, dim3(grid > 0 ? grid : 1), dim3(64), 0, static_cast<hipStream_t>(stream));
    return (int)hipGetLastError();
}

}  // extern "C"
