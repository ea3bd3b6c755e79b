// Small-batch (M = 1..16) GEMV C ABI on the matrix cores: variant tables, argument checks, launch.
//
// No reference symbol: the reference's kernels are M = 1 only, and M = 1..16 is its open item (src/README.md:118)
// that its harness sweeps for library GEMMs (paia-bench/configs/shapes.yaml:63-64). The entry points take the same
// weight operands and follow the same conventions as the M = 1 entry points (src/paia_gemv/gemv_quant.cu:59-99):
// rc 0 ok, -1 bad variant, -2 bad shape or alignment, > 0 a hipError_t; caller-owned device memory, no allocation, no
// synchronisation. x is bf16 [M][K] and y bf16 [M][N], both row-major.
//
// Variant knobs: P tiles of 16 rows per wave, U k-blocks (128 columns) of loads in flight per wave, W waves per block,
// S waves sharing a tile along K (split-K inside the block). variant < 0 selects paia_gemv_batch_pick_variant's.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_batch.h"
#include "paia_gemv.h"

namespace {
using namespace paia;

template <int F, int P, int U, int W>
int launch_b(BatchParams p, hipStream_t st)
{
    return launch_batch<F, P, U, W>(p, st);
}

#define BV(F, P, U, W, S) {P, U, W, S, &launch_b<F, P, U, W>},
#define BV_W(F, P, U) BV(F, P, U, 4, 1) BV(F, P, U, 4, 2) BV(F, P, U, 4, 4) \
                      BV(F, P, U, 8, 1) BV(F, P, U, 8, 2) BV(F, P, U, 8, 4) BV(F, P, U, 8, 8)
// register budget: P * U * (16-byte loads per k-block) <= 16 buffers of 4 VGPRs
const BatchVariant kBf16Batch[] = {BV_W(kBF16, 1, 2) BV_W(kBF16, 1, 4) BV_W(kBF16, 2, 2)};
const BatchVariant kFp8Batch[] = {BV_W(kFP8, 1, 2) BV_W(kFP8, 1, 4) BV_W(kFP8, 1, 8) BV_W(kFP8, 2, 2)
                                      BV_W(kFP8, 2, 4) BV_W(kFP8, 4, 2)};
const BatchVariant kI4Batch[] = {BV_W(kI4, 1, 4) BV_W(kI4, 1, 8) BV_W(kI4, 2, 2) BV_W(kI4, 2, 4) BV_W(kI4, 2, 8)
                                     BV_W(kI4, 4, 2) BV_W(kI4, 4, 4)};
const BatchVariant kI4ZpBatch[] = {BV_W(kI4ZP, 1, 4) BV_W(kI4ZP, 1, 8) BV_W(kI4ZP, 2, 2) BV_W(kI4ZP, 2, 4)
                                       BV_W(kI4ZP, 2, 8) BV_W(kI4ZP, 4, 2) BV_W(kI4ZP, 4, 4)};
#undef BV
#undef BV_W

struct Table {
    const BatchVariant* v;
    int n;
};
Table table(int kind)
{
    switch (kind) {
    case 0: return {kBf16Batch, (int)(sizeof(kBf16Batch) / sizeof(kBf16Batch[0]))};
    case 1: return {kFp8Batch, (int)(sizeof(kFp8Batch) / sizeof(kFp8Batch[0]))};
    case 2: return {kI4Batch, (int)(sizeof(kI4Batch) / sizeof(kI4Batch[0]))};
    case 3: return {kI4ZpBatch, (int)(sizeof(kI4ZpBatch) / sizeof(kI4ZpBatch[0]))};
    default: return {nullptr, 0};
    }
}

int find(const Table& t, int P, int U, int W, int S)
{
    for (int i = 0; i < t.n; ++i)
        if (t.v[i].P == P && t.v[i].U == U && t.v[i].W == W && t.v[i].S == S) return i;
    return -1;
}

// LDS bytes a variant needs for this shape (0 if no chunk fits), computed like batch_plan.
uint32_t plan_lds(int kind, int M, int K, int P, int U, int W, int S)
{
    const int KB = (K + kBlockCols - 1) / kBlockCols;
    const int kbs = (KB + S - 1) / S;
    const bool i4 = kind >= 2;
    const uint32_t per_kb = (uint32_t)(S * M) * 256u + (i4 ? (uint32_t)S * 64u : 0u);
    const uint32_t fixed = (uint32_t)(S * M) * 16u;
    if (fixed + per_kb * (uint32_t)U > kBatchLds) return 0;
    int C = (int)((kBatchLds - fixed) / per_kb);
    C -= C % U;
    const int cap = (kbs + U - 1) / U * U;
    if (C > cap) C = cap;
    const uint32_t xb = fixed + per_kb * (uint32_t)C;
    const uint32_t pb = S > 1 ? (uint32_t)((W / S) * (S - 1) * P) * 1024u : 0u;
    return xb > pb ? xb : pb;
}

// Default choice: the format's tile/pipeline shape, then the fewest K-splits that put at least ~8 waves on every CU
// (at least 4 k-blocks per split, and the x chunk must fit).
int pick(int kind, int M, int N, int K)
{
    const Table t = table(kind);
    if (!t.v || M < 1 || M > kMaxBatch || N <= 0 || K <= 0) return -1;
    int P = 2, U = 4, W = 4;
    if (kind == 0) {
        P = 1;
        U = 4;
    }
    const int ntiles = (N + kTileRows - 1) / kTileRows;
    const int KB = (K + kBlockCols - 1) / kBlockCols;
    const DeviceFacts df = device_facts();
    const int want = (df.cus > 0 ? df.cus : 256) * 8;
    int best = -1;
    for (int S = 1; S <= 4; S *= 2) {
        if (S > 1 && (KB + S - 1) / S < 4) break;
        if (plan_lds(kind, M, K, P, U, W, S) == 0) break;
        best = find(t, P, U, W, S);
        if ((ntiles + P - 1) / P * S >= want) break;
    }
    if (best < 0) {
        // large M x K: the smallest pipeline that fits
        for (int i = 0; i < t.n && best < 0; ++i)
            if (t.v[i].S == 1 && plan_lds(kind, M, K, t.v[i].P, t.v[i].U, t.v[i].W, 1) != 0) best = i;
    }
    return best;
}

int batch_impl(int kind, BatchParams p, int variant, void* stream)
{
    const Table t = table(kind);
    if (variant < 0) variant = pick(kind, p.M, p.N, p.K);
    if (variant < 0 || variant >= t.n) return -1;
    p.S = t.v[variant].S;
    return t.v[variant].fn(p, static_cast<hipStream_t>(stream));
}

// Shared checks: 1 <= M <= 16, N, K > 0, K bounded so a 16-row tile's bytes fit one buffer descriptor, x 16-byte and
// y 2-byte aligned, bias 2-byte aligned.
bool common_ok(const void* x, const void* y, const void* bias, int M, int N, int K)
{
    return M >= 1 && M <= kMaxBatch && N > 0 && K > 0 && K <= (1 << 24) && aligned(x, 16) && aligned(y, 2) &&
           (!bias || aligned(bias, 2));
}

}  // namespace

extern "C" {

int paia_gemv_batch_variant_count(int kind) { return table(kind).n; }

int paia_gemv_batch_variant_info(int kind, int v, int* P, int* U, int* W, int* S)
{
    const Table t = table(kind);
    if (v < 0 || v >= t.n) return -1;
    *P = t.v[v].P;
    *U = t.v[v].U;
    *W = t.v[v].W;
    *S = t.v[v].S;
    return 0;
}

int paia_gemv_batch_pick_variant(int kind, int M, int N, int K) { return pick(kind, M, N, K); }

int paia_gemv_batch_bf16(const void* W, const void* x, const void* bias, void* y, int M, int N, int K, int variant,
                         void* stream)
{
    if (variant >= table(0).n) return -1;
    if (!common_ok(x, y, bias, M, N, K) || (K & 7) || !aligned(W, 16)) return -2;
    BatchParams p{};
    p.W = static_cast<const uint8_t*>(W);
    p.x = static_cast<const uint16_t*>(x);
    p.bias = static_cast<const uint16_t*>(bias);
    p.y = static_cast<uint16_t*>(y);
    p.M = M;
    p.N = N;
    p.K = K;
    p.row_bytes = (uint32_t)K * 2u;
    return batch_impl(0, p, variant, stream);
}

int paia_gemv_batch_fp8(const void* Wq, const void* scale, const void* x, const void* bias, void* y, int M, int N,
                        int K, int variant, void* stream)
{
    if (variant >= table(1).n) return -1;
    if (!common_ok(x, y, bias, M, N, K) || (K & 15) || !aligned(Wq, 16) || !aligned(scale, 4)) return -2;
    BatchParams p{};
    p.W = static_cast<const uint8_t*>(Wq);
    p.meta = scale;
    p.x = static_cast<const uint16_t*>(x);
    p.bias = static_cast<const uint16_t*>(bias);
    p.y = static_cast<uint16_t*>(y);
    p.M = M;
    p.N = N;
    p.K = K;
    p.row_bytes = (uint32_t)K;
    return batch_impl(1, p, variant, stream);
}

int paia_gemv_batch_int4(const void* Wq, const void* scales, const void* x, void* y, int M, int N, int K, int variant,
                         void* stream)
{
    if (variant >= table(2).n) return -1;
    if (!common_ok(x, y, nullptr, M, N, K) || (K & 127) || !aligned(Wq, 16) || !aligned(scales, 2)) return -2;
    BatchParams p{};
    p.W = static_cast<const uint8_t*>(Wq);
    p.meta = scales;
    p.x = static_cast<const uint16_t*>(x);
    p.y = static_cast<uint16_t*>(y);
    p.M = M;
    p.N = N;
    p.K = K;
    p.row_bytes = (uint32_t)K / 2u;
    p.meta_bytes = (uint32_t)(K / 128) * 2u;
    return batch_impl(2, p, variant, stream);
}

int paia_gemv_batch_int4_zp(const void* Wq, const void* scales, const void* zeros, const void* x, const void* bias,
                            void* y, int M, int N, int K, int variant, void* stream)
{
    if (variant >= table(3).n) return -1;
    if (!common_ok(x, y, bias, M, N, K) || (K & 127) || !aligned(Wq, 16) || !aligned(scales, 2) || !zeros) return -2;
    BatchParams p{};
    p.W = static_cast<const uint8_t*>(Wq);
    p.meta = scales;
    p.zeros = static_cast<const uint8_t*>(zeros);
    p.x = static_cast<const uint16_t*>(x);
    p.bias = static_cast<const uint16_t*>(bias);
    p.y = static_cast<uint16_t*>(y);
    p.M = M;
    p.N = N;
    p.K = K;
    p.row_bytes = (uint32_t)K / 2u;
    p.meta_bytes = (uint32_t)(K / 128) * 2u;
    p.zbytes = (uint32_t)((K / 128 + 1) / 2);
    return batch_impl(3, p, variant, stream);
}

}  // extern "C"
