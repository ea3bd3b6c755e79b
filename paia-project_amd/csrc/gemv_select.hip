// Per-shape variant choice for gfx950 (used when a caller passes variant = -1 to the torch ops).
// No reference C symbol: the reference picks variants in Python from src/tuned/<platform>.json
// (paia-bench/bench/ops/ours_bf16.py:32-38, ours_quant.py:29-36); this is the same idea compiled into the library so
// the torch ops need no JSON. A shape without an entry takes the entry of the nearest tuned shape of its format
// (smallest |log2(N/N')| + |log2(K/K')|), and only a format with no entry at all the harness default tuples
// (ours_bf16.py:22, ours_quant.py:19): measured on MI355X, the split-K default runs large untuned shapes ~15% slower
// than their tuned neighbours' choice (BF16 131072x4096: 74.6% of 8 TB/s, against 90.8% for the tuned 128256x4096).
//
// The table is data, not code: paia-project_amd/tuned/mi355x.json keeps the reference's tuned-file schema
// ("shapes" / "fp8_shapes" / "int4_shapes" keyed "NxK", plus "int4zp_shapes"), written by paia_bench.sweep
// --write-tuned on an MI355X; build.py turns it into gemv_tuned.inc.
#include <hip/hip_runtime.h>

#include <cmath>

#include "gemv_kernel.h"
#include "paia_gemv.h"

namespace {

struct Pick {
    int kind, N, K, R, U, W, S, H;
};

// kind: 0 BF16, 1 FP8, 2 INT4 (reference format), 3 INT4 asymmetric. Generated at build time from
// paia-project_amd/tuned/mi355x.json (the MI355X sweep's frozen per-shape choices) by build.py.
const Pick kTuned[] = {
#include "gemv_tuned.inc"
    {-1, 0, 0, 0, 0, 0, 0, 0},   // end marker
};

// Whether a variant of table 0 (BF16), 1 (FP8) or 2 (INT4, both formats) stages x for this K in the LDS: the launch's
// LDS plan (paia::lds_plan, the one the launch itself goes by) fits x and the INT4 lane sums plus, for split-K, one
// round of partial sums. A variant that does not runs the x-from-global kernel instead, which is slower, so the pick
// prefers one that does.
bool stages_x(int table, int R, int W, int H, int K)
{
    using namespace paia;
    const uint64_t row_bytes = table == 0 ? 2ull * (uint64_t)K : table == 1 ? (uint64_t)K : (uint64_t)K / 2u;
    const uint64_t nchunks = (row_bytes + kChunkBytes - 1) / kChunkBytes;
    if (nchunks > (uint64_t)(kMaxLds / kChunkBytes)) return false;   // cannot fit at any format: skip the plan
    int round = 0;
    return lds_plan(table == 0 ? kBF16 : table == 1 ? kFP8 : kI4, R, W, H != 0, (int)nchunks, &round) != 0;
}

int find_bf16(int R, int U, int W, int S, int H)
{
    for (int i = 0; i < paia_gemv_bf16_variant_count(); ++i) {
        int r, u, w, s, h;
        paia_gemv_bf16_variant_info(i, &r, &u, &w, &s, &h);
        if (r == R && u == U && w == W && s == S && h == H) return i;
    }
    return -1;
}

int find_quant(int kind, int R, int U, int W, int H)
{
    const int n = kind == 1 ? paia_gemv_fp8_variant_count() : paia_gemv_int4_variant_count();
    for (int i = 0; i < n; ++i) {
        int r, u, w, h;
        if (kind == 1) paia_gemv_fp8_variant_info(i, &r, &u, &w, &h);
        else paia_gemv_int4_variant_info(i, &r, &u, &w, &h);
        if (r == R && u == U && w == W && h == H) return i;
    }
    return -1;
}

}  // namespace

extern "C" {

int paia_gemv_pick_variant(int kind, int N, int K)
{
    if (kind < 0 || kind > 3) kind = 0;
    const int table = kind == 3 ? 2 : kind;   // both INT4 formats use the paia_gemv_int4 variant table
    // a tuned entry counts only where its x fits the LDS at this K (a split-K entry needs room for its partials too)
    auto resolve = [&](const Pick& p) {
        if (!stages_x(table, p.R, p.W, p.H, K)) return -1;
        return table == 0 ? find_bf16(p.R, p.U, p.W, p.S, p.H) : find_quant(table, p.R, p.U, p.W, p.H);
    };
    for (int pass = 0; pass < 2; ++pass) {    // this kind's row first; the asymmetric INT4 falls back to INT4's
        const int want = pass == 0 ? kind : (kind == 3 ? 2 : -2);
        for (const Pick& p : kTuned) {
            if (p.kind == want && p.N == N && p.K == K) {
                const int v = resolve(p);
                if (v >= 0) return v;
            }
        }
    }
    if (N > 0 && K > 0) {
        for (int pass = 0; pass < 2; ++pass) {
            const int want = pass == 0 ? kind : (kind == 3 ? 2 : -2);
            int best = -1;
            double best_d = 0.0;
            for (const Pick& p : kTuned) {
                if (p.kind != want || p.N <= 0 || p.K <= 0) continue;
                const double d = std::fabs(std::log2((double)N / p.N)) + std::fabs(std::log2((double)K / p.K));
                const int v = resolve(p);
                if (v >= 0 && (best < 0 || d < best_d)) {
                    best = v;
                    best_d = d;
                }
            }
            if (best >= 0) return best;
        }
    }
    // the harness default tuple, or its row-parallel twin where the split-K partials do not fit; at K beyond any
    // staging, every variant runs the same x-from-global kernel
    int R = 2, U = 4, W = 4, H = 1;
    if (table == 1) U = 2;
    else if (table == 2) R = 4, U = 2;
    if (!stages_x(table, R, W, H, K)) H = 0;
    const int v = table == 0 ? find_bf16(R, U, W, 0, H) : find_quant(table, R, U, W, H);
    return v < 0 ? 0 : v;
}

// Which kernel a launch of `variant` runs at (N, K): 0 gemv_kernel, 1 gemv_kernel43 (INT4 with few weight loads per
// wave: the 0x43-exponent decode), 2 gemv_kernel_xg (K beyond the LDS), 3 gemv_kernel_dr / 4 gemv_kernel43_dr (0 / 1
// ending in a drain: at most two items per wave), as a profiler names them; -1 bad kind or variant, -2 bad shape. No
// launch; the grid sizing queries the current device once.
int paia_gemv_launch_kind(int kind, int N, int K, int variant)
{
    if (kind < 0 || kind > 3) return -1;
    if (N <= 0 || K <= 0) return -2;
    paia::GemvParams p{};
    p.N = N;
    p.K = K;
    const int G = K / 128;
    switch (kind) {
    case 0:
        p.row_bytes = 2u * (uint32_t)K;
        return paia::kind_bf16(variant, p);
    case 1:
        p.row_bytes = (uint32_t)K;
        return paia::kind_fp8(variant, p);
    default:
        if (K & 127) return -2;
        p.row_bytes = (uint32_t)K / 2u;
        p.meta_bytes = (uint32_t)G * 2u;
        p.zbytes = kind == 3 ? (uint32_t)(G + 1) / 2u : 0u;
        return paia::kind_int4(variant, kind == 3, p);
    }
}

}  // extern "C"
