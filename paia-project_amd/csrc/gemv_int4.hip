// INT4 W4A16 group-128 GEMV C ABI.
//
// Reference format (drop-in for src/paia_gemv/gemv_quant.cu:70-97): nibbles n in [N][K/2] (byte j = weights 2j low,
// 2j+1 high; on a little-endian machine identical to "8 per int32 along K"), zero point 8, fp16 scale [N][K/128]:
//   paia_gemv_int4          fused kernel, variant table (R,U,W,H)
//   paia_gemv_int4_naive    the deliberately naive control (one row per wave, 4-byte loads, per-weight decode)
//   paia_gemv_int4_unfused  the unfused control: dequantise to a caller-owned bf16 scratch, then the BF16 GEMV
// Asymmetric format (no reference counterpart; BASELINE INT4 configs): q in 0..15, bf16 scale [N][G], 4-bit zero
// point per group packed 2 per byte along G ([N][ceil(G/2)], group 2j low nibble), optional bf16 bias:
//   paia_gemv_int4_zp       fused kernel, same variant table as paia_gemv_int4
//
// Variant knobs on gfx950: R rows per wave {1,2,4,8}, U 16-byte loads per row per batch {1,2,4}, W waves per block
// {4,8}, H split-K inside the block {0,1}; plus W = 16 (one block per CU) with R {1,2}, U {1,2,4}, H 0; plus U 1, H 0
// with (R, W) (1,9), (2,9), (1,12), (1,14) (whole blocks per CU on the small BASELINE shapes). Weight loads are always
// "nt" (S reported as 0).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "gemv_kernel.h"
#include "paia_gemv.h"

namespace paia {

// K1 naive control. One row per wave, each lane loads 4 bytes (8 weights) per iteration, reloads the group scale from
// memory every iteration and decodes each weight with shift/mask/convert. Kept simple on purpose (no LDS, no
// batching) so it measures what the fused design buys. Semantics follow src/paia_gemv/gemv_int4.cuh:125-152.
__global__ void __launch_bounds__(256) gemv_int4_naive_kernel(const uint8_t* __restrict__ Wq,
                                                              const uint16_t* __restrict__ scales,
                                                              const uint16_t* __restrict__ x,
                                                              uint16_t* __restrict__ y, int N, int K)
{
    const int lane = lane_id();
    const int row = (int)blockIdx.x * 4 + wave_id();
    if (row >= N) return;
    const uint32_t* wr = reinterpret_cast<const uint32_t*>(Wq + (size_t)row * (size_t)(K / 2));
    const uint16_t* sr = scales + (size_t)row * (size_t)(K / 128);
    float acc = 0.0f;
#pragma unroll 1
    for (int col = lane * 8; col < K; col += 512) {
        const uint32_t w = wr[col >> 3];
        const float s = f16_to_f32(sr[col >> 7]);
        const u32x4 xv = *reinterpret_cast<const u32x4*>(x + col);
        const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int n = (int)((w >> (4 * j)) & 0xFu);
            const float xf = (j & 1) ? bf16_to_f32(xw[j >> 1] >> 16) : bf16_to_f32(xw[j >> 1] & 0xFFFFu);
            acc = __builtin_fmaf((float)(n - 8) * s, xf, acc);
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = (uint16_t)f32_to_bf16_rne(acc);
}

// Unfused control, stage 1 (src/paia_gemv/gemv_int4.cuh:155-174): bf16 copy bf16_rn((n - 8) * s) of the weights.
// One thread handles 8 weights (one 32-bit word) per iteration and writes 16 bytes.
__global__ void __launch_bounds__(256) dequant_int4_bf16_kernel(const uint8_t* __restrict__ Wq,
                                                                const uint16_t* __restrict__ scales,
                                                                uint16_t* __restrict__ out, size_t n_words, int K)
{
    const size_t words_per_row = (size_t)K / 8;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words; i += (size_t)gridDim.x * blockDim.x) {
        const uint32_t w = reinterpret_cast<const uint32_t*>(Wq)[i];
        const size_t row = i / words_per_row;
        const int k = (int)(i - row * words_per_row) * 8;
        const float s = f16_to_f32(scales[row * (size_t)(K / 128) + (size_t)(k >> 7)]);
        u32x4 o;
        uint32_t* po = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float a = (float)((int)((w >> (8 * j)) & 0xFu) - 8) * s;
            const float b = (float)((int)((w >> (8 * j + 4)) & 0xFu) - 8) * s;
            po[j] = f32_to_bf16_rne(a) | (f32_to_bf16_rne(b) << 16);
        }
        *reinterpret_cast<u32x4*>(out + i * 8) = o;
    }
}

}  // namespace paia

namespace {
using namespace paia;

constexpr int kQuantAux = 2;   // nt: weights are streamed once per call

template <int F, int R, int U, int W, int H>
int launch_i4(GemvParams p, hipStream_t st)
{
    return launch_gemv<F, R, U, W, kQuantAux, H != 0>(p, st);
}

template <int F, int R, int U, int W, int H>
int kind_of_i4(GemvParams p)
{
    return gemv_kernel_kind<F, R, U, W, kQuantAux, H != 0>(p);
}

#define QV(R, U, W, H) {R, U, W, 0, H, &launch_i4<kI4, R, U, W, H>, &kind_of_i4<kI4, R, U, W, H>},
#define QV_W(R, U, H) QV(R, U, 4, H) QV(R, U, 8, H)
#define QV_H(R, U) QV_W(R, U, 0) QV_W(R, U, 1)
#define QV_U(R) QV_H(R, 1) QV_H(R, 2) QV_H(R, 4)
// one 16-wave block per CU (row-parallel only), appended so the indices above stay stable
#define QV_16 QV(1, 1, 16, 0) QV(1, 2, 16, 0) QV(1, 4, 16, 0) QV(2, 1, 16, 0) QV(2, 2, 16, 0) QV(2, 4, 16, 0)
// block sizes that make the small BASELINE shapes a whole number of blocks per CU (row-parallel only; appended after
// the W = 16 ones): 4608 rows in 512 blocks of 9 (R = 1) or 256 of 9 (R = 2), 6144 rows in 512 blocks of 12, 3584
// rows in 256 blocks of 14
#define QV_WB QV(1, 1, 9, 0) QV(2, 1, 9, 0) QV(1, 1, 12, 0) QV(1, 1, 14, 0)
const Variant kInt4Variants[] = {QV_U(1) QV_U(2) QV_U(4) QV_U(8) QV_16 QV_WB};
#undef QV
#define QV(R, U, W, H) {R, U, W, 0, H, &launch_i4<kI4ZP, R, U, W, H>, &kind_of_i4<kI4ZP, R, U, W, H>},
const Variant kInt4ZpVariants[] = {QV_U(1) QV_U(2) QV_U(4) QV_U(8) QV_16 QV_WB};
#undef QV
#undef QV_W
#undef QV_H
#undef QV_U
#undef QV_16
#undef QV_WB
constexpr int kNumInt4 = (int)(sizeof(kInt4Variants) / sizeof(kInt4Variants[0]));
static_assert(sizeof(kInt4Variants) == sizeof(kInt4ZpVariants), "int4 tables must match");

bool int4_args_ok(const void* Wq, const void* scales, const void* x, const void* y, int N, int K)
{
    return N > 0 && K > 0 && (K & 127) == 0 && aligned(Wq, 16) && aligned(x, 16) && aligned(scales, 2) &&
           aligned(y, 2);
}

// R=2 U=4 W=4 S=0 H=1, looked up by its knobs (as src/paia_gemv/gemv_quant.cu:47-56 does).
int default_bf16_variant()
{
    static const int v = [] {   // thread-safe one-time initialisation
        for (int i = 0; i < paia_gemv_bf16_variant_count(); ++i) {
            int R, U, W, S, H;
            paia_gemv_bf16_variant_info(i, &R, &U, &W, &S, &H);
            if (R == 2 && U == 4 && W == 4 && S == 0 && H == 1) return i;
        }
        return 0;
    }();
    return v;
}

// ---- the unfused control without a caller workspace (paia_gemv_int4_unfused_noalloc) ------------------------------
// Scratch for the dequantised bf16 rows: a static device array (each GPU the library runs on holds its own copy from
// module load to process exit). Host code never passes the array's name to a kernel (on the host it is only a
// stand-in symbol): the device address comes from hipGetSymbolAddress, taken once per device with that device
// current, on the entry point's first call there.
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_dev[kMaxDevices];
std::mutex g_scratch_mu;

// The current device's address of `scratch` (0 and *rc = 0 on success, else *rc = the hipError_t or -2).
void* scratch_device_ptr(int* rc)
{
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        *rc = (int)e;
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        *rc = -2;
        return nullptr;
    }
    void* p = g_scratch_dev[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_dev[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            const hipError_t g = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (g != hipSuccess || p == nullptr) {
                *rc = g != hipSuccess ? (int)g : (int)hipErrorInvalidSymbol;
                return nullptr;
            }
            g_scratch_dev[dev].store(p, std::memory_order_release);
        }
    }
    *rc = 0;
    return p;
}

// Rows per slice: as many whole 8-row blocks of bf16 rows as the scratch holds (8 keeps every slice's y and Wq
// offsets 16-byte aligned). 0 when not even 8 rows fit (K > 2097152).
int noalloc_slice_rows(int K)
{
    const size_t row = (size_t)K * 2u;
    const size_t rows = kNoAllocScratchBytes / row;
    return (int)(rows / 8u * 8u);
}

}  // namespace

namespace paia {
int launch_gemv_int4_picked(GemvParams p, bool zp, hipStream_t st)
{
    const int v = paia_gemv_pick_variant(zp ? 3 : 2, p.N, p.K);
    return (zp ? kInt4ZpVariants : kInt4Variants)[v].fn(p, st);
}
int kind_int4(int v, bool zp, GemvParams p)
{
    return v < 0 || v >= kNumInt4 ? -1 : (zp ? kInt4ZpVariants : kInt4Variants)[v].kind(p);
}
}  // namespace paia

extern "C" {

int paia_gemv_int4_variant_count() { return kNumInt4; }

int paia_gemv_int4_variant_info(int v, int* R, int* U, int* W, int* H)
{
    if (v < 0 || v >= kNumInt4) return -1;
    *R = kInt4Variants[v].R;
    *U = kInt4Variants[v].U;
    *W = kInt4Variants[v].W;
    *H = kInt4Variants[v].H;
    return 0;
}

int paia_gemv_int4(const void* Wq, const void* scales, const void* x, void* y, int N, int K, int variant, void* stream)
{
    if (variant < 0 || variant >= kNumInt4) return -1;
    if (!int4_args_ok(Wq, scales, x, y, N, K)) return -2;
    GemvParams p{};
    p.W = static_cast<const uint8_t*>(Wq);
    p.meta = scales;
    p.x = static_cast<const uint16_t*>(x);
    p.y = static_cast<uint16_t*>(y);
    p.N = N;
    p.K = K;
    p.row_bytes = (uint32_t)K / 2u;
    p.meta_bytes = (uint32_t)(K / 128) * 2u;
    return kInt4Variants[variant].fn(p, static_cast<hipStream_t>(stream));
}

int paia_gemv_int4_zp(const void* Wq, const void* scales, const void* zeros, const void* x, const void* bias, void* y,
                      int N, int K, int variant, void* stream)
{
    if (variant < 0 || variant >= kNumInt4) return -1;
    if (!int4_args_ok(Wq, scales, x, y, N, K) || zeros == nullptr || (bias && !aligned(bias, 2))) return -2;
    const int G = K / 128;
    GemvParams p{};
    p.W = static_cast<const uint8_t*>(Wq);
    p.meta = scales;
    p.zeros = static_cast<const uint8_t*>(zeros);
    p.x = static_cast<const uint16_t*>(x);
    p.bias = static_cast<const uint16_t*>(bias);
    p.y = static_cast<uint16_t*>(y);
    p.N = N;
    p.K = K;
    p.row_bytes = (uint32_t)K / 2u;
    p.meta_bytes = (uint32_t)G * 2u;
    p.zbytes = (uint32_t)(G + 1) / 2u;
    return kInt4ZpVariants[variant].fn(p, static_cast<hipStream_t>(stream));
}

int paia_gemv_int4_naive(const void* Wq, const void* scales, const void* x, void* y, int N, int K, void* stream)
{
    if (!int4_args_ok(Wq, scales, x, y, N, K)) return -2;
    hipLaunchKernelGGL(gemv_int4_naive_kernel, dim3((N + 3) / 4), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint8_t*>(Wq), static_cast<const uint16_t*>(scales),
                       static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), N, K);
    return (int)hipGetLastError();
}

int paia_gemv_int4_unfused_noalloc(const void* Wq, const void* scales, const void* x, void* y, int N, int K,
                                   void* stream)
{
    if (N <= 0 || K <= 0 || (K & 127) || !aligned(Wq, 16) || !aligned(x, 16) || !aligned(scales, 2) ||
        !aligned(y, 16))
        return -2;
    const int slice = noalloc_slice_rows(K);
    if (slice < 8) return -2;   // K beyond the scratch: 8 bf16 rows of K values must fit kNoAllocScratchBytes
    int rc = 0;
    void* sp = scratch_device_ptr(&rc);
    if (sp == nullptr) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int variant = default_bf16_variant();
    const size_t wrow = (size_t)K / 2u, srow = (size_t)K / 128u;
    // slice by slice on the caller's stream: dequantise rows [n0, n0 + n) into the scratch, then the BF16 GEMV of
    // those rows into y[n0 ..]; the next slice's dequantisation is ordered after this GEMV, which has then read it.
    // Each output row depends only on its own row and the variant, so the result equals paia_gemv_int4_unfused's.
    for (int n0 = 0; n0 < N; n0 += slice) {
        const int n = N - n0 < slice ? N - n0 : slice;
        const size_t words = (size_t)n * (size_t)K / 8;
        const size_t want = (words + 255) / 256;
        const unsigned grid = (unsigned)(want < 8192 ? want : 8192);
        hipLaunchKernelGGL(dequant_int4_bf16_kernel, dim3(grid), dim3(256), 0, st,
                           static_cast<const uint8_t*>(Wq) + (size_t)n0 * wrow,
                           static_cast<const uint16_t*>(scales) + (size_t)n0 * srow, static_cast<uint16_t*>(sp), words,
                           K);
        rc = (int)hipGetLastError();
        if (rc) return rc;
        rc = paia_gemv_bf16(sp, x, static_cast<uint16_t*>(y) + n0, n, K, variant, stream);
        if (rc) return rc;
    }
    return 0;
}

int paia_gemv_int4_unfused(const void* Wq, const void* scales, const void* x, void* y, void* scratch_bf16, int N, int K,
                           void* stream)
{
    if (N <= 0 || K <= 0 || (K & 127) || !aligned(Wq, 16) || !aligned(x, 16) || !aligned(scales, 2) ||
        !aligned(scratch_bf16, 16))
        return -2;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t words = (size_t)N * (size_t)K / 8;
    const size_t want = (words + 255) / 256;
    const unsigned grid = (unsigned)(want < 8192 ? want : 8192);
    hipLaunchKernelGGL(dequant_int4_bf16_kernel, dim3(grid), dim3(256), 0, st, static_cast<const uint8_t*>(Wq),
                       static_cast<const uint16_t*>(scales), static_cast<uint16_t*>(scratch_bf16), words, K);
    const int rc = (int)hipGetLastError();
    if (rc) return rc;
    return paia_gemv_bf16(scratch_bf16, x, y, N, K, default_bf16_variant(), stream);
}

}  // extern "C"
