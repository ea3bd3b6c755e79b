// Measurement kernels for the benchmark harness (libpaia_probe.so; not part of the GEMV library).
//
// paia_probe_read: a pure streaming read, 16-byte nontemporal loads with a grid-stride loop and an XOR sink that
//   keeps the loads alive -- the MI355X counterpart of the reference's dev read probe "B0"
//   (src/tests/gemv_bf16_check.cu:131-139,228-252). Timing it on the same byte counts as a GEMV gives the achievable
//   bandwidth (and the fixed cost) that kernel is measured against.
// paia_probe_stream: the same read through the GEMV's own load path: raw buffer loads (16 bytes per lane, nt) of
//   1-KiB chunks, U chunks per item, two items in flight per wave, items dealt round-robin to the waves of a
//   persistent grid of blocks_per_cu blocks of W waves on every CU (the walk of the fused GEMV at R = 1, H = 0,
//   without x, the decode or the store). The benchmark takes the best of both probes, over their launch shapes, as
//   the read floor.
// paia_probe_stream_lead: the same read in 8-wave blocks of which only wave 0 streams (items dealt round-robin to the
//   blocks), the walk of a split-K GEMV launch whose rows are one segment long.
// paia_probe_set_output: makes the read probes also write a GEMV's output, nout bf16 values (0: none, the default),
//   each thread or wave its equal share when its reads are done (the cheapest time to write them: a GEMV that writes
//   a row group's outputs as the group completes cannot do better). The benchmark's "I/O floor" of a GEMV: its
//   weight bytes read and its outputs written.
// paia_probe_read_staged: the grid-stride read (unroll 1) of 256-thread blocks that each first stage xbytes of a
//   second buffer into LDS behind a block barrier, as every block of a GEMV stages x before its first item, and read
//   one staged vector per loaded one. The floor of a read that must stage x first: what a GEMV of these bytes and
//   this K (xbytes = 2K) cannot beat with x in LDS.
// paia_probe_copy: a plain 16-byte-per-lane copy of known size, the calibration kernel for the rocprofv3 byte counters
//   (FETCH_SIZE should read its size once, WRITE_SIZE its size once).
// paia_probe_empty: an empty kernel, for the per-launch floor of back-to-back launches in a graph.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int UNROLL, bool OUT>
__global__ void __launch_bounds__(256) read_probe_kernel(const u32x4* __restrict__ p, size_t n16, uint32_t* sink,
                                                         uint16_t* y, uint32_t nout)
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
    if (OUT)
        for (size_t j = (size_t)blockIdx.x * blockDim.x + threadIdx.x; j < nout; j += stride) y[j] = (uint16_t)acc;
}

constexpr uint32_t kOOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t nbytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes, 0x00020000);
}

// Reads nbytes (< 2^31) once. Item i = bytes [i*U KiB, (i+1)*U KiB): wave w of block b takes items b*W + w + k*grid*W.
// Two item buffers, each refilled right after it is consumed; items past the end load at an out-of-range offset (no
// traffic). The loop is left by `return` when a wave's items run out, as the GEMV's loop is. The loads come from
// read-only memory, so the compiler may move them to their first use (then only one item is in flight): an empty
// asm barrier after each issue keeps them in place, and the exit folds both buffers (zeros there) into the sink.
// LEAD: only wave 0 of each block streams, taking items blockIdx.x + k*gridDim.x; the other waves return at once.
// OUT: streaming wave gw of nw writes outputs [gw*nout/nw, (gw+1)*nout/nw) when its items are done.
template <int U, int W, bool LEAD, bool OUT>
__global__ void __launch_bounds__(W * 64) stream_probe_kernel(const void* __restrict__ buf, uint32_t nbytes,
                                                              uint32_t* sink, uint16_t* y, uint32_t nout)
{
    const __amdgpu_buffer_rsrc_t r = make_rsrc(buf, nbytes);
    const uint32_t lane16 = (threadIdx.x & 63u) * 16u;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if (LEAD && wave != 0) return;
    constexpr uint32_t item_bytes = U * 1024u;
    const uint32_t nitems = (nbytes + item_bytes - 1) / item_bytes;
    uint32_t item = LEAD ? blockIdx.x : blockIdx.x * W + wave;
    const uint32_t stride = LEAD ? gridDim.x : gridDim.x * W;
    uint32_t acc = 0;
    u32x4 b[2][U];
    bool valid[2];
    auto issue = [&](int d) {
        valid[d] = item < nitems;
        const uint32_t off = valid[d] ? item * item_bytes + lane16 : kOOB;
#pragma unroll
        for (int u = 0; u < U; ++u)
            b[d][u] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off + u * 1024u, 0u, 2));
        item += stride;
        asm volatile("" ::: "memory");   // compiler barrier: the loads stay where they are issued (no sinking)
    };
    const uint32_t first = item;   // the wave's index among the streaming waves (its first item)
    auto consume = [&](int d) {
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= b[d][u].x ^ b[d][u].y ^ b[d][u].z ^ b[d][u].w;
    };
    issue(0);
    issue(1);
    // one exit test per trip (two would merge into one exit block whose false edge reaches the loop header, and the
    // wait counts would then assume the newest loads are the ones consumed first); the trip's second item may lie
    // past the end: its loads return zeros without traffic
    for (;;) {
        if (!valid[0]) {
            consume(0);
            consume(1);
            if (acc == 0x9E3779B9u) sink[0] = acc;   // practically never true; keeps the loads alive
            if (OUT) {
                const uint32_t o1 = (uint32_t)((uint64_t)(first + 1) * nout / stride);
                for (uint32_t o = (uint32_t)((uint64_t)first * nout / stride) + (threadIdx.x & 63u); o < o1; o += 64u)
                    y[o] = (uint16_t)acc;
            }
            return;
        }
        consume(0);
        __builtin_amdgcn_sched_barrier(0);   // keep each refill after the consume of its buffer
        issue(0);
        __builtin_amdgcn_sched_barrier(0);
        consume(1);
        __builtin_amdgcn_sched_barrier(0);
        issue(1);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The output paia_probe_set_output installed (none by default).
uint16_t* g_out_y = nullptr;
uint32_t g_out_n = 0;

template <int U, int W, bool LEAD = false>
int launch_stream(const void* buf, uint32_t nbytes, uint32_t* sink, int grid, hipStream_t st)
{
    if (g_out_n == 0) {
        hipLaunchKernelGGL((stream_probe_kernel<U, W, LEAD, false>), dim3(grid), dim3(W * 64), 0, st, buf, nbytes, sink,
                           nullptr, 0u);
        return (int)hipGetLastError();
    }
    hipLaunchKernelGGL((stream_probe_kernel<U, W, LEAD, true>), dim3(grid), dim3(W * 64), 0, st, buf, nbytes, sink,
                       g_out_y, g_out_n);
    return (int)hipGetLastError();
}

__global__ void __launch_bounds__(256) copy_probe_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                         size_t n16)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

__global__ void __launch_bounds__(256) staged_read_kernel(const u32x4* __restrict__ p, size_t n16, uint32_t* sink,
                                                          const u32x4* __restrict__ x, uint32_t nx16)
{
    extern __shared__ u32x4 xs[];
    for (uint32_t j = threadIdx.x; j < nx16; j += blockDim.x) xs[j] = x[j];
    __syncthreads();
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    uint32_t j = threadIdx.x % nx16;   // the staged vector read with each load: walks x, 64 vectors a step
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const u32x4 v = __builtin_nontemporal_load(p + i);
        const u32x4 xv = xs[j];
        j += 64u;
        j = j >= nx16 ? j - nx16 : j;   // nx16 >= 64, so one subtraction keeps j < nx16
        acc ^= (v.x ^ v.y ^ v.z ^ v.w) + (xv.x ^ xv.w);
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;   // practically never true; keeps the loads alive
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
    uint16_t* y = g_out_y;
    const uint32_t no = g_out_n;
#define READ_CASE(UN)                                                                                              \
    case UN:                                                                                                       \
        if (no) hipLaunchKernelGGL((read_probe_kernel<UN, true>), dim3(grid), dim3(256), 0, st, p, n16, s, y, no); \
        else hipLaunchKernelGGL((read_probe_kernel<UN, false>), dim3(grid), dim3(256), 0, st, p, n16, s, y, no);   \
        break;
    switch (unroll) {
    READ_CASE(1) READ_CASE(4) READ_CASE(8)
    default: return -1;
    }
#undef READ_CASE
    return (int)hipGetLastError();
}

// x: xbytes (1024..65536, a multiple of 16, 16-byte aligned) staged into LDS by every block first.
__attribute__((visibility("default"))) int paia_probe_read_staged(const void* buf, size_t nbytes, void* sink, int grid,
                                                                  const void* x, int xbytes, void* stream)
{
    if (!buf || !sink || !x || (reinterpret_cast<uintptr_t>(buf) & 15) || (reinterpret_cast<uintptr_t>(x) & 15) ||
        grid <= 0 || xbytes < 1024 || xbytes > 65536 || (xbytes & 15))
        return -2;
    hipLaunchKernelGGL(staged_read_kernel, dim3(grid), dim3(256), (uint32_t)xbytes, static_cast<hipStream_t>(stream),
                       static_cast<const u32x4*>(buf), nbytes / 16, static_cast<uint32_t*>(sink),
                       static_cast<const u32x4*>(x), (uint32_t)xbytes / 16u);
    return (int)hipGetLastError();
}

// U in {1, 2, 4, 8} with W in {4, 8, 16}, and U = 16 with W in {4, 8}; grid = blocks (the caller passes CUs x blocks
// per CU); nbytes < 2^31.
__attribute__((visibility("default"))) int paia_probe_stream(const void* buf, size_t nbytes, void* sink, int U, int W,
                                                             int grid, void* stream)
{
    const bool shape_ok = ((U == 1 || U == 2 || U == 4 || U == 8) && (W == 4 || W == 8 || W == 16)) ||
                          (U == 16 && (W == 4 || W == 8));
    if (!shape_ok) return -1;   // checked first, so a caller can test a shape with null buffers
    if (!buf || !sink || (reinterpret_cast<uintptr_t>(buf) & 15) || grid <= 0 || nbytes == 0 || nbytes >= (1ull << 31))
        return -2;
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint32_t* s = static_cast<uint32_t*>(sink);
    const uint32_t n = (uint32_t)nbytes;
#define PROBE_CASE(UU, WW) \
    if (U == UU && W == WW) return launch_stream<UU, WW>(buf, n, s, grid, st);
#define PROBE_W(UU) PROBE_CASE(UU, 4) PROBE_CASE(UU, 8) PROBE_CASE(UU, 16)
    PROBE_W(1) PROBE_W(2) PROBE_W(4) PROBE_W(8) PROBE_CASE(16, 4) PROBE_CASE(16, 8)   // 16 KiB items at W = 16 spill
#undef PROBE_W
#undef PROBE_CASE
    return -1;
}

// 8-wave blocks whose wave 0 streams U-KiB items (U in {8, 16}); grid = blocks; nbytes < 2^31.
__attribute__((visibility("default"))) int paia_probe_stream_lead(const void* buf, size_t nbytes, void* sink, int U,
                                                                  int grid, void* stream)
{
    if (U != 8 && U != 16) return -1;   // checked first, so a caller can test a shape with null buffers
    if (!buf || !sink || (reinterpret_cast<uintptr_t>(buf) & 15) || grid <= 0 || nbytes == 0 || nbytes >= (1ull << 31))
        return -2;
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint32_t* s = static_cast<uint32_t*>(sink);
    const uint32_t n = (uint32_t)nbytes;
    return U == 8 ? launch_stream<8, 8, true>(buf, n, s, grid, st) : launch_stream<16, 8, true>(buf, n, s, grid, st);
}

// y: nout bf16 values (nout < 2^31); nout = 0 (y ignored) turns the writes off.
__attribute__((visibility("default"))) int paia_probe_set_output(void* y, size_t nout)
{
    if (nout >= (1ull << 31) || (nout && (!y || (reinterpret_cast<uintptr_t>(y) & 1)))) return -2;
    g_out_y = nout ? static_cast<uint16_t*>(y) : nullptr;
    g_out_n = (uint32_t)nout;
    return 0;
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
