// Small-batch (M = 1..16) GEMV C ABI: variant tables (matrix-core, row-streaming and M = 1 entries), argument checks,
// pick, launch.
//
// No reference symbol: the reference's kernels are M = 1 only, and M = 1..16 is its open item (src/README.md:118)
// that its harness sweeps for library GEMMs (paia-bench/configs/shapes.yaml:63-64). The entry points take the same
// weight operands and follow the same conventions as the M = 1 entry points (src/paia_gemv/gemv_quant.cu:59-99):
// rc 0 ok, -1 bad variant, -2 bad shape or alignment, > 0 a hipError_t; caller-owned device memory, no allocation, no
// synchronisation. x is bf16 [M][K] and y bf16 [M][N], both row-major.
//
// Variant knobs: P tiles of 16 rows per wave, U k-blocks (128 columns) of loads in flight per wave, W waves per block,
// S waves sharing a tile along K (split-K inside the block), X how x reaches the matrix cores (0 staged in LDS per
// K-chunk of up to 64 KiB, 1 loaded with the weights, 2 staged as for 0 in chunks of up to 80 KiB, or the device's
// per-block LDS if less). variant < 0 selects paia_gemv_batch_pick_variant's.
//
// P = 0 marks the row-streaming kernel instead (gemv_rows_kernel: the M = 1 GEMV's weight stream and decode with one
// accumulator per activation row, for M = 2..6, BF16 and FP8 also 7, 8): then U is its 1-KiB chunks per item, W its waves per
// block, S its weight rows per wave (R) and X the one M it serves (other M: -2). These entries follow the matrix-core
// ones.
// The last entry, P = U = W = S = 0 and X = 1, is the M = 1 GEMV itself (the M = 1 entry point's kernel and variant
// choice) and serves M = 1 only.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_batch.h"
#include "gemv_kernel.h"
#include "paia_gemv.h"

namespace {
using namespace paia;

// LDS budget of the X = 2 variants on this device
uint32_t wide_lds() { return rows_max_lds() < kBatchLdsWide ? rows_max_lds() : kBatchLdsWide; }

template <int F, int P, int U, int W, int X>
int launch_b(BatchParams p, hipStream_t st)
{
    if constexpr (X == 2) return launch_batch<F, P, U, W, 0>(p, st, wide_lds());
    return launch_batch<F, P, U, W, X>(p, st);
}

GemvParams gemv_params(const BatchParams& b)
{
    GemvParams p{};
    p.W = b.W;
    p.meta = b.meta;
    p.zeros = b.zeros;
    p.x = b.x;
    p.bias = b.bias;
    p.y = b.y;
    p.N = b.N;
    p.K = b.K;
    p.row_bytes = b.row_bytes;
    p.meta_bytes = b.meta_bytes;
    p.zbytes = b.zbytes;
    return p;
}

// the row-streaming kernel for exactly MB activation rows (weights streamed once: nt loads)
template <int F, int R, int U, int W, int MB>
int launch_rows_b(BatchParams b, hipStream_t st)
{
    if (b.M != MB) return -2;
    return launch_gemv_rows<F, R, U, W, 2, MB>(gemv_params(b), st);
}

// M = 1: the M = 1 GEMV with the library's M = 1 variant
template <int F>
int launch_m1_b(BatchParams b, hipStream_t st)
{
    if (b.M != 1) return -2;
    const GemvParams p = gemv_params(b);
    if (F == kBF16) return launch_gemv_bf16_picked(p, st);
    if (F == kFP8) return launch_gemv_fp8_picked(p, st);
    return launch_gemv_int4_picked(p, F == kI4ZP, st);
}

#define BV(F, P, U, W, S, X) {P, U, W, S, X, &launch_b<F, P, U, W, X>},
#define RV(F, R, U, W, MB) {0, U, W, R, MB, &launch_rows_b<F, R, U, W, MB>},
#define M1V(F) {0, 0, 0, 0, 1, &launch_m1_b<F>},
#define RV_M(F, R, U, W) RV(F, R, U, W, 2) RV(F, R, U, W, 3) RV(F, R, U, W, 4)
#define RV_ALL(F) RV_M(F, 1, 2, 8) RV_M(F, 2, 2, 4) RV_M(F, 1, 1, 8) RV_M(F, 2, 1, 4) RV_M(F, 1, 2, 16) \
                  RV_M(F, 2, 1, 16)
// M = 5..8, BF16 and FP8 (INT4: 5, 6): BF16 has no decode (4 v_dot2 per 16 weight bytes and activation row), so 8 rows
// stay within the VALU budget and the default pick streams them; FP8 and INT4 spend most of their VALU at M = 4 on the
// tall shapes, so only a measured entry (the tuned table) picks these for them, where they beat the matrix cores
#define RV_M8(F, R, U, W) RV(F, R, U, W, 5) RV(F, R, U, W, 6) RV(F, R, U, W, 7) RV(F, R, U, W, 8)
// INT4 at M = 5, 6 (seven and eight rows of staged x and lane sums do not fit the 16-wave launch's 128 VGPRs)
#define RV_M6(F, R, U, W) RV(F, R, U, W, 5) RV(F, R, U, W, 6)
#define RV_ALL6(F) RV_M6(F, 1, 2, 8) RV_M6(F, 2, 2, 4) RV_M6(F, 1, 1, 8) RV_M6(F, 2, 1, 4) RV_M6(F, 1, 2, 16) \
                   RV_M6(F, 2, 1, 16)
#define RV_ALL8(F) RV_M8(F, 1, 2, 8) RV_M8(F, 2, 2, 4) RV_M8(F, 1, 1, 8) RV_M8(F, 2, 1, 4) RV_M8(F, 1, 2, 16) \
                   RV_M8(F, 2, 1, 16)
#define BV_S(F, P, U, X) BV(F, P, U, 4, 1, X) BV(F, P, U, 4, 2, X) BV(F, P, U, 4, 4, X) \
                         BV(F, P, U, 8, 1, X) BV(F, P, U, 8, 2, X) BV(F, P, U, 8, 4, X) BV(F, P, U, 8, 8, X)
#define BV_W(F, P, U) BV_S(F, P, U, 0) BV_S(F, P, U, 1) BV_S(F, P, U, 2)
// register budget: P * U * (16-byte loads per k-block) <= 16 buffers of 4 VGPRs (INT4 P=2 U=8 with x loaded
// alongside spilled, so it is left out)
const BatchVariant kBf16Batch[] = {BV_W(kBF16, 1, 2) BV_W(kBF16, 1, 4) BV_W(kBF16, 2, 2) RV_ALL(kBF16)
                                       RV_ALL8(kBF16) M1V(kBF16)};
const BatchVariant kFp8Batch[] = {BV_W(kFP8, 1, 2) BV_W(kFP8, 1, 4) BV_W(kFP8, 1, 8) BV_W(kFP8, 2, 2)
                                      BV_W(kFP8, 2, 4) BV_W(kFP8, 4, 2) RV_ALL(kFP8) RV_ALL8(kFP8) M1V(kFP8)};
const BatchVariant kI4Batch[] = {BV_W(kI4, 1, 4) BV_W(kI4, 1, 8) BV_W(kI4, 2, 2) BV_W(kI4, 2, 4) BV_W(kI4, 4, 2)
                                     BV_W(kI4, 4, 4) RV_ALL(kI4) RV_ALL6(kI4) M1V(kI4)};
const BatchVariant kI4ZpBatch[] = {BV_W(kI4ZP, 1, 4) BV_W(kI4ZP, 1, 8) BV_W(kI4ZP, 2, 2) BV_W(kI4ZP, 2, 4)
                                       BV_W(kI4ZP, 4, 2) BV_W(kI4ZP, 4, 4) RV_ALL(kI4ZP) RV_ALL6(kI4ZP)
                                       M1V(kI4ZP)};
#undef BV
#undef BV_S
#undef BV_W
#undef RV
#undef RV_M
#undef RV_ALL
#undef RV_M8
#undef RV_ALL8
#undef RV_M6
#undef RV_ALL6
#undef M1V

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

int find(const Table& t, int P, int U, int W, int S, int X)
{
    for (int i = 0; i < t.n; ++i)
        if (t.v[i].P == P && t.v[i].U == U && t.v[i].W == W && t.v[i].S == S && t.v[i].X == X) return i;
    return -1;
}

// Whether variant v can run (M, K): X=0 needs a chunk of U k-blocks of x for all S splits in LDS; a row-streaming
// variant (and the M = 1 entry) serves its own M only (its LDS limit is checked at launch).
bool fits(const BatchVariant& v, int M)
{
    if (v.P == 0) return v.X == M;
    return v.X == 1 || batch_x_bytes(v.S, M, v.U) <= (v.X == 2 ? wide_lds() : kBatchLds);
}

// Default choice: a measured entry for the shape and M when the tuned table has one; otherwise a rule fitted to MI355X
// sweeps of the Llama/Qwen projection shapes (FP8 and INT4). M = 1 takes the M = 1 GEMV when its staged x fits the LDS
// (it beat the matrix-core kernel on every BASELINE shape: FP8 gate_up 18.9 µs against 22.7, INT4 asymmetric 12.2
// against 16.5). M = 2..4 (BF16 2..8) take the row-streaming kernel when its x copies fit the LDS (pick_rows; BF16 at
// M = 5..8 measured 9-37% faster than the matrix cores on every BASELINE shape where it fits); otherwise the
// matrix-core kernel:
//   * split-K S: at least two splits (every shape streamed faster with two waves per tile than with one), then the
//     fewest (<= 8, >= 2 k-blocks each) that give >= 1152 work units (tiles x splits, 4.5 per CU): qkv (384 tiles)
//     measured best at S = 4, o/down (256 tiles) at S = 8, gate_up (1792 tiles) at S = 2;
//   * x in LDS (X=0) unless the splits x rows make staging cost more than it saves (M*S >= 24 with S >= 4: each block
//     would stage a third or more of its weight bytes again as x; measured at M = 3 on the tall-K down shapes, whose
//     three x copies do not fit the row-streaming kernel: X=0 20.1 µs against 16.1 for X=1 at M = 4) or not even
//     one chunk of U k-blocks fits;
//   * one tile per wave; two when x comes with the weights and M >= 8, so the two tiles share each x load, provided
//     the halved tile count still gives >= 1152 units within 8 splits (at 256 tiles it does not, and one tile per
//     wave was faster there);
//   * x with the weights at M >= 8: four waves per block and at most four splits.
constexpr int kPickUnits = 1152;

int pick_splits(int units0, int KB, int W)
{
    int S = 1;
    while (S < W && (S == 1 || units0 * S < kPickUnits) && (KB + 2 * S - 1) / (2 * S) >= 2) S *= 2;
    return S;
}

// LDS of the row-streaming kernel at M activation rows: M staged copies of x (+ INT4 lane sums), and for INT4 the
// per-wave |x| maxima of a block of up to 16 waves (kind is the format number).
uint64_t rows_lds(int kind, int M, int K)
{
    const uint64_t row_bytes = kind == 0 ? 2ull * K : (kind == 1 ? (uint64_t)K : (uint64_t)K / 2);
    const uint64_t nchunks = (row_bytes + kChunkBytes - 1) / kChunkBytes;
    const uint64_t xq = kind == 0 ? 1 : (kind == 1 ? 2 : 4);
    return (uint64_t)M * nchunks * (xq * kChunkBytes + (kind >= 2 ? kWave * 4u : 0u)) + lds_slot_bytes(kind, M, 16);
}

// The row-streaming variant for M = 2..4 (BF16 2..8): the M = 1 tuned choice's (R, U, W) when the table has that
// triple (the weight stream is the M = 1 kernel's), else R=1 U=2 W=8. -1 when its x copies do not fit the LDS.
int pick_rows(const Table& t, int kind, int M, int N, int K)
{
    if (M < 2 || M > (kind == 0 ? 8 : 4) || rows_lds(kind, M, K) > rows_max_lds()) return -1;
    // INT4 at M = 4 on tall N: the four v_dot2 chains per decoded word saturate the VALU; the matrix cores were
    // faster there (gate_up 28672x4096: 17.4 µs against 20.4; Qwen gate_up: 20.5 against 24.5)
    if (kind >= 2 && M >= 4 && N >= 16384) return -1;
    int R = 1, U = 2, W = 8;
    const int v1 = paia_gemv_pick_variant(kind, N, K);
    int r = 0, u = 0, w = 0, s = 0, h = 1;
    const int rc = kind == 0 ? paia_gemv_bf16_variant_info(v1, &r, &u, &w, &s, &h)
                             : (kind == 1 ? paia_gemv_fp8_variant_info(v1, &r, &u, &w, &h)
                                          : paia_gemv_int4_variant_info(v1, &r, &u, &w, &h));
    if (rc == 0 && h == 0 && find(t, 0, u, w, r, M) >= 0) {
        R = r;
        U = u;
        W = w;
    }
    return find(t, 0, U, W, R, M);
}

// Measured choices for the BASELINE shapes (tuned/mi355x.json's "*batch_shapes" sections, compiled in by build.py).
struct BatchPick {
    int kind, M, N, K, P, U, W, S, X;
};
const BatchPick kBatchTuned[] = {
#include "gemv_batch_tuned.inc"
    {-1, 0, 0, 0, 0, 0, 0, 0, 0},   // end marker
};

int pick(int kind, int M, int N, int K)
{
    const Table t = table(kind);
    if (!t.v || M < 1 || M > kMaxBatch || N <= 0 || K <= 0) return -1;
    for (const BatchPick& b : kBatchTuned)
        if (b.kind == kind && b.M == M && b.N == N && b.K == K) {
            const int v = find(t, b.P, b.U, b.W, b.S, b.X);
            // a row-streaming entry also needs its x copies to fit this device's LDS (the entries were measured with
            // MI355X's 160 KiB per block)
            const bool lds_ok = b.P != 0 || b.U == 0 || rows_lds(kind, M, K) <= rows_max_lds();
            if (v >= 0 && fits(t.v[v], M) && lds_ok) return v;
        }
    // the M = 1 GEMV's x (+ INT4 lane sums) and room for its split-K partials (W*R floats, <= 512 bytes)
    if (M == 1 && rows_lds(kind, 1, K) + 512 <= kMaxLds) return find(t, 0, 0, 0, 0, 1);
    const int rv = pick_rows(t, kind, M, N, K);
    if (rv >= 0) return rv;
    int W = 8;
    const int ntiles = (N + kTileRows - 1) / kTileRows;
    const int KB = (K + kBlockCols - 1) / kBlockCols;
    const int U = kind >= 2 ? 4 : 2;
    int S = pick_splits(ntiles, KB, W);
    int P = 1, X = 0;
    if ((M * S >= 24 && S >= 4) || batch_x_bytes(S, M, U) > kBatchLds) X = 1;
    if (X == 1 && M >= 8) {
        const int pairs = (ntiles + 1) / 2;
        const int S2 = pick_splits(pairs, KB, W);
        if (pairs * S2 >= kPickUnits) {
            P = 2;
            S = S2;
        }
    }
    // M >= 8 with x loaded alongside the weights: four waves sharing a tile in at most four splits (measured on every
    // INT4 and BF16 projection shape but gate_up at M = 8 and 16: 3-9% faster than eight waves in eight splits; FP8
    // within 0.4% or faster)
    if (X == 1 && M >= 8) {
        W = 4;
        S = S < 4 ? S : 4;
    }
    return find(t, P, U, W, S, X);
}

int batch_impl(int kind, BatchParams p, int variant, void* stream)
{
    const Table t = table(kind);
    if (variant < 0) variant = pick(kind, p.M, p.N, p.K);
    if (variant < 0 || variant >= t.n) return -1;
    if (!fits(t.v[variant], p.M)) return -2;
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

int paia_gemv_batch_variant_info(int kind, int v, int* P, int* U, int* W, int* S, int* X)
{
    const Table t = table(kind);
    if (v < 0 || v >= t.n) return -1;
    *P = t.v[v].P;
    *U = t.v[v].U;
    *W = t.v[v].W;
    *S = t.v[v].S;
    *X = t.v[v].X;
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
