// FP8 W8A16 GEMV C ABI: variant table, argument checks, launch.
// Drop-in for src/paia_gemv/gemv_quant.cu:61-68 (same symbols, return codes and argument contract).
//
// Weights are OCP e4m3fn bytes [N][K] with one fp32 scale per row: y[n] = bf16_rn(scale[n] * sum_k e4m3(W[n,k]) x[k]).
// The decode is gfx950's e4m3 -> bf16 pair convert (v_cvt_scalef32_pk_bf16_fp8 at scale 1, exact for every code).
// Codes 0x7F/0xFF are NaN in e4m3fn and decode to NaN here, as the reference's dequantiser defines them
// (quant_host.h:19, quant.py:16-17); the quantiser never emits them.
//
// Variant knobs on gfx950 (reference tuple shape R,U,W,H; S is reported as 0 and the loads are always "nt"):
//   R rows per wave {1,2,4}, U 16-byte loads per row per batch {1,2,4}, W waves per block {4,8},
//   H split-K inside the block {0,1}; plus W = 16 (one block per CU) with R {1,2}, U {1,2,4}, H 0; plus R 1, U 2,
//   W {6,12}, H 0 (whole blocks per CU on the small BASELINE shapes).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_kernel.h"
#include "paia_gemv.h"

namespace {
using namespace paia;

constexpr int kQuantAux = 2;   // nt: weights are streamed once per call

template <int R, int U, int W, int H>
int launch_fp8(GemvParams p, hipStream_t st)
{
    return launch_gemv<kFP8, R, U, W, kQuantAux, H != 0>(p, st);
}

template <int R, int U, int W, int H>
int kind_of_fp8(GemvParams p)
{
    return gemv_kernel_kind<kFP8, R, U, W, kQuantAux, H != 0>(p);
}

#define QV(R, U, W, H) {R, U, W, 0, H, &launch_fp8<R, U, W, H>, &kind_of_fp8<R, U, W, H>},
#define QV_W(R, U, H) QV(R, U, 4, H) QV(R, U, 8, H)
#define QV_H(R, U) QV_W(R, U, 0) QV_W(R, U, 1)
#define QV_U(R) QV_H(R, 1) QV_H(R, 2) QV_H(R, 4)
// one 16-wave block per CU (row-parallel only), appended so the indices above stay stable
#define QV_16 QV(1, 1, 16, 0) QV(1, 2, 16, 0) QV(1, 4, 16, 0) QV(2, 1, 16, 0) QV(2, 2, 16, 0) QV(2, 4, 16, 0)
// block sizes that make the small BASELINE shapes a whole number of blocks per CU (row-parallel only; appended after
// the W = 16 ones): 4608 rows in 768 blocks of 6, 6144 rows in 512 blocks of 12
#define QV_WB QV(1, 2, 6, 0) QV(1, 2, 12, 0)
const Variant kFp8Variants[] = {QV_U(1) QV_U(2) QV_U(4) QV_16 QV_WB};
#undef QV
#undef QV_W
#undef QV_H
#undef QV_U
#undef QV_16
#undef QV_WB
constexpr int kNumFp8 = (int)(sizeof(kFp8Variants) / sizeof(kFp8Variants[0]));

int gemv_fp8_impl(const void* Wq, const void* scale, const void* x, const void* bias, void* y, int N, int K,
                  int variant, void* stream)
{
    if (variant < 0 || variant >= kNumFp8) return -1;
    if (N <= 0 || K <= 0 || (K & 15) != 0) return -2;
    if (!aligned(Wq, 16) || !aligned(x, 16) || !aligned(scale, 4) || !aligned(y, 2) || (bias && !aligned(bias, 2)))
        return -2;
    GemvParams p{};
    p.W = static_cast<const uint8_t*>(Wq);
    p.meta = scale;
    p.x = static_cast<const uint16_t*>(x);
    p.bias = static_cast<const uint16_t*>(bias);
    p.y = static_cast<uint16_t*>(y);
    p.N = N;
    p.K = K;
    p.row_bytes = (uint32_t)K;
    return kFp8Variants[variant].fn(p, static_cast<hipStream_t>(stream));
}

}  // namespace

namespace paia {
int launch_gemv_fp8_picked(GemvParams p, hipStream_t st)
{
    return kFp8Variants[paia_gemv_pick_variant(1, p.N, p.K)].fn(p, st);
}
int kind_fp8(int v, GemvParams p)
{
    return v < 0 || v >= kNumFp8 ? -1 : kFp8Variants[v].kind(p);
}
}  // namespace paia

extern "C" {

int paia_gemv_fp8_variant_count() { return kNumFp8; }

int paia_gemv_fp8_variant_info(int v, int* R, int* U, int* W, int* H)
{
    if (v < 0 || v >= kNumFp8) return -1;
    *R = kFp8Variants[v].R;
    *U = kFp8Variants[v].U;
    *W = kFp8Variants[v].W;
    *H = kFp8Variants[v].H;
    return 0;
}

int paia_gemv_fp8(const void* Wq, const void* scale, const void* x, void* y, int N, int K, int variant, void* stream)
{
    return gemv_fp8_impl(Wq, scale, x, nullptr, y, N, K, variant, stream);
}

int paia_gemv_fp8_bias(const void* Wq, const void* scale, const void* x, const void* bias, void* y, int N, int K,
                       int variant, void* stream)
{
    return gemv_fp8_impl(Wq, scale, x, bias, y, N, K, variant, stream);
}

}  // extern "C"
