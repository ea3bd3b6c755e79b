// Per-shape variant choice for gfx950 (used when a caller passes variant = -1 to the torch ops).
// No reference C symbol: the reference picks variants in Python from src/tuned/<platform>.json
// (paia-bench/bench/ops/ours_bf16.py:32-38, ours_quant.py:29-36); this is the same idea compiled into the library so
// the torch ops need no JSON. Shapes without an entry use the harness default tuples (ours_bf16.py:22,
// ours_quant.py:19).
#include <hip/hip_runtime.h>

#include "paia_gemv.h"

namespace {

struct Pick {
    int kind, N, K, R, U, W, S, H;
};

// kind: 0 BF16, 1 FP8, 2 INT4 (both INT4 formats share a table)
const Pick kTuned[] = {
    {0, 0, 0, 2, 4, 4, 0, 1},   // placeholder row: defaults until the MI355X sweep fills this table
};

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
    for (const Pick& p : kTuned) {
        if (p.kind == kind && p.N == N && p.K == K) {
            const int v = kind == 0 ? find_bf16(p.R, p.U, p.W, p.S, p.H) : find_quant(kind, p.R, p.U, p.W, p.H);
            if (v >= 0) return v;
        }
    }
    int v = -1;
    if (kind == 0) v = find_bf16(2, 4, 4, 0, 1);
    else if (kind == 1) v = find_quant(1, 2, 2, 4, 1);
    else v = find_quant(2, 4, 2, 4, 1);
    return v < 0 ? 0 : v;
}

}  // extern "C"
