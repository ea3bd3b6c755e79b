// BF16 GEMV C ABI: variant table, argument checks, launch.
// Drop-in for src/paia_gemv/gemv_bf16.cu:35-55 (same symbols, same return codes and argument contract).
//
// Variant knobs on gfx950 (the tuple space keeps the reference's shape so tuned tables and harness defaults carry
// over; the meaning is the gfx950 one):
//   R  rows per wave {1,2,4}        U  16-byte loads per row per batch {1,2,4,8} (two batches are in flight)
//   W  waves per block {4,8}        S  nontemporal ("nt") weight loads {0,1}
//   H  split-K inside the block {0,1}: the W waves share R rows and split the row's chunks
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_kernel.h"
#include "paia_gemv.h"

namespace {
using namespace paia;

template <int R, int U, int W, int S, int H>
int launch_bf16(GemvParams p, hipStream_t st)
{
    return launch_gemv<kBF16, R, U, W, S ? 2 : 0, H != 0>(p, st);
}

template <int R, int U, int W, int S, int H>
int kind_of_bf16(GemvParams p)
{
    return gemv_kernel_kind<kBF16, R, U, W, S ? 2 : 0, H != 0>(p);
}

#define PV(R, U, W, S, H) {R, U, W, S, H, &launch_bf16<R, U, W, S, H>, &kind_of_bf16<R, U, W, S, H>},
#define PV_W(R, U, S, H) PV(R, U, 4, S, H) PV(R, U, 8, S, H)
#define PV_H(R, U, S) PV_W(R, U, S, 0) PV_W(R, U, S, 1)
#define PV_S(R, U) PV_H(R, U, 0) PV_H(R, U, 1)
#define PV_U(R) PV_S(R, 1) PV_S(R, 2) PV_S(R, 4) PV_S(R, 8)
const Variant kBf16Variants[] = {PV_U(1) PV_U(2) PV_U(4)};
#undef PV
#undef PV_W
#undef PV_H
#undef PV_S
#undef PV_U
constexpr int kNumBf16 = (int)(sizeof(kBf16Variants) / sizeof(kBf16Variants[0]));

int gemv_bf16_impl(const void* W, const void* x, const void* bias, void* y, int N, int K, int variant, void* stream)
{
    if (variant < 0 || variant >= kNumBf16) return -1;
    if (N <= 0 || K <= 0 || (K & 7) != 0) return -2;
    if (!aligned(W, 16) || !aligned(x, 16) || !aligned(y, 16) || (bias && !aligned(bias, 2))) return -2;
    GemvParams p{};
    p.W = static_cast<const uint8_t*>(W);
    p.x = static_cast<const uint16_t*>(x);
    p.bias = static_cast<const uint16_t*>(bias);
    p.y = static_cast<uint16_t*>(y);
    p.N = N;
    p.K = K;
    p.row_bytes = (uint32_t)K * 2u;
    return kBf16Variants[variant].fn(p, static_cast<hipStream_t>(stream));
}

}  // namespace

namespace paia {
int launch_gemv_bf16_picked(GemvParams p, hipStream_t st)
{
    return kBf16Variants[paia_gemv_pick_variant(0, p.N, p.K)].fn(p, st);
}
int kind_bf16(int v, GemvParams p)
{
    return v < 0 || v >= kNumBf16 ? -1 : kBf16Variants[v].kind(p);
}
}  // namespace paia

extern "C" {

int paia_gemv_bf16_variant_count() { return kNumBf16; }

int paia_gemv_bf16_variant_info(int v, int* R, int* U, int* W, int* S, int* H)
{
    if (v < 0 || v >= kNumBf16) return -1;
    *R = kBf16Variants[v].R;
    *U = kBf16Variants[v].U;
    *W = kBf16Variants[v].W;
    *S = kBf16Variants[v].S;
    *H = kBf16Variants[v].H;
    return 0;
}

int paia_gemv_bf16(const void* W, const void* x, void* y, int N, int K, int variant, void* stream)
{
    return gemv_bf16_impl(W, x, nullptr, y, N, K, variant, stream);
}

int paia_gemv_bf16_bias(const void* W, const void* x, const void* bias, void* y, int N, int K, int variant,
                        void* stream)
{
    return gemv_bf16_impl(W, x, bias, y, N, K, variant, stream);
}

}  // extern "C"
