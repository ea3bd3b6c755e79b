// Small-batch GEMV for gfx950 on the matrix cores: M = 1..16 activation rows against one weight matrix.
//
//   y[m, n] = bf16_rn( sum_k deq(W[n,k]) * x[m,k]  (+ bias[n]) ),   x bf16 [M][K], y bf16 [M][N]
//
// The reference's kernels are M = 1 only; M = 1..16 is its open item (src/README.md:118) and the M sweep of its
// harness (paia-bench/configs/shapes.yaml:63-64, bench/run.py:88-91). Same weight formats and semantics as the M = 1
// kernel, with the products on MFMA instead of v_dot2:
//   * One v_mfma_f32_16x16x32_bf16 takes A = x (16 activation rows x 32 columns, bf16) and B = dequantised weights
//     (32 columns x 16 output rows, bf16) and accumulates D[m][n] in fp32. Lane l supplies A row l%16 and B column
//     l%16, eight consecutive k each, from k-group l/16; it holds D rows 4*(l/16)+v, v = 0..3, of column l%16. Rows
//     m >= M of A repeat row 0 and their D rows are never stored (MFMA rows are independent).
//   * Tile = 16 weight rows. A k-block = 128 columns = 4 MFMA steps. Per tile and k-block a lane issues L = 1 (INT4),
//     2 (FP8) or 4 (BF16) 16-byte buffer loads; load i of lane group h covers bytes 64i + 16h .. +15 of the row's
//     k-block, so each load instruction reads 64 contiguous bytes of 16 rows.
//   * Dequantisation in registers as in the M = 1 kernel: FP8 by the gfx950 e4m3 -> f32 convert packed to bf16 (exact),
//     INT4 by v_perm of the nibbles under a 0x43 byte, giving bf16 (128 + q) exactly; the INT4 group term
//     (128 + z) * sum_k x[m,k] is removed per group, with the group sums of x taken by one more MFMA chain against a
//     B operand of ones (it lands in the lanes and rows of D that need it, shared by the wave's P tiles).
//   * x (the A operand) comes one of two ways (knob X):
//       X=0: staged in LDS per K-chunk of up to 64 KiB (all of K when M*K fits, as at M = 1) in the column order the
//            format's MFMA steps take (INT4: (k, k+2, k+4, k+6, k+1, k+3, k+5, k+7) within each 8, matching the
//            nibble decode); a chunk change costs two block barriers and drains the load pipeline. X=2 is the same
//            kernel with chunks of up to 80 KiB (fewer chunk changes; the launch raises the LDS limit).
//       X=1: loaded per k-block straight into registers with the weights (L2-resident: x is at most 16 rows), in the
//            same pipeline; no LDS, no barrier, no K limit -- the choice for many rows or long K.
//   * Each wave owns P tiles and one of S K-splits; the S waves sharing a tile combine their fp32 partials through
//     LDS in split order after a block barrier, so results are bitwise reproducible. U k-blocks of loads are in flight
//     per wave; the loads of the next k-blocks are issued before the current ones are consumed.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "gemv_device.h"
#include "gemv_kernel.h"

namespace paia {


constexpr int kTileRows = 16;    // weight rows per MFMA tile
constexpr int kBlockCols = 128;  // columns per k-block (4 MFMA steps of 32; one INT4 group)
constexpr int kMaxBatch = 16;    // activation rows per call

// Cache policy of the weight loads (buffer-load aux bits). 0, the default policy: measured on MI355X ~10% faster
// than nt (2) for this kernel's 64-byte-per-row load pattern (FP8 gate_up 28672x4096: 22.1 vs 24.5 us at M = 1).
#ifndef PAIA_BATCH_WAUX
#define PAIA_BATCH_WAUX 0
#endif

template <int F>
struct BatchFmt {
    // weight bytes per row per k-block, and 16-byte loads per lane per tile per k-block
    static constexpr int kBytesKB = F == kBF16 ? 256 : (F == kFP8 ? 128 : 64);
    static constexpr int kLoads = kBytesKB / 64;
};

struct BatchParams {
    const uint8_t* W;       // weight rows, row_bytes each
    const void* meta;       // FP8: fp32 scale [N]; INT4: fp16 scale [N][G]; INT4ZP: bf16 scale [N][G]
    const uint8_t* zeros;   // INT4ZP: [N][zbytes] packed 4-bit zero points
    const uint16_t* x;      // bf16 [M][K]
    const uint16_t* bias;   // bf16 [N] or null
    uint16_t* y;            // bf16 [M][N]
    int M, N, K;
    uint32_t row_bytes;     // weight bytes per row
    uint32_t meta_bytes;    // INT4: scale bytes per row (2 G)
    uint32_t zbytes;        // INT4ZP: zero-point bytes per row (ceil(G/2))
    int KB;                 // k-blocks: ceil(K / 128)
    int ntiles;             // ceil(N / 16)
    int S;                  // K-splits per tile (waves sharing a tile); divides W
    int kbs;                // k-blocks per split: ceil(KB / S)
    int C;                  // k-blocks per LDS chunk of each split (a multiple of U)
    int nchunks;            // ceil(kbs / C)
    uint32_t xrow;          // X=0: LDS bytes per staged x row: C*256 + 16 (the 16 spreads rows over the banks)
};

// First column (within a k-block) of the 8 that MFMA step j takes from lane group h; the other steps' columns follow
// from the byte layout of the loads (load i of group h = bytes 64i + 16h .. +15 of the row's k-block).
template <int F>
__host__ __device__ constexpr int step_col(int j, int h)
{
    return F == kBF16 ? 32 * j + 8 * h : (F == kFP8 ? 64 * (j >> 1) + 16 * h + 8 * (j & 1) : 32 * h + 8 * j);
}

// LDS layout of a launch: X=0 x chunk [S][M][xrow], reused for the split-K partials after the last chunk.
__host__ __device__ constexpr uint32_t batch_x_bytes(int S, int M, int C)
{
    return (uint32_t)(S * M) * (uint32_t)(C * 256 + 16);
}
__host__ __device__ constexpr uint32_t batch_part_bytes(int S, int W, int P)
{
    return S > 1 ? (uint32_t)((W / S) * (S - 1) * P) * 1024u : 0u;
}

// INT4 x vector (x0..x7 as bf16 pairs) re-paired to the nibble decode order (x0,x2),(x4,x6),(x1,x3),(x5,x7).
__device__ __forceinline__ u32x4 i4_pair_x(const u32x4 a)
{
    return u32x4{__builtin_amdgcn_perm(a.y, a.x, 0x05040100u), __builtin_amdgcn_perm(a.w, a.z, 0x05040100u),
                 __builtin_amdgcn_perm(a.y, a.x, 0x07060302u), __builtin_amdgcn_perm(a.w, a.z, 0x07060302u)};
}

// MG (INT4): metadata grouping. MG=1 loads each group's scale (and zero point) with the group's k-block. MG=4 loads
// them for four groups at once (8 bytes of scales, 2 bytes of zero points per row), with the k-block whose stage is a
// multiple of 4: each such load touches 16 rows' cache lines, so a quarter of them cuts the kernel's memory
// instructions per k-block from 3 to 1.5 (measured: INT4 gate_up 23.6 -> 17.3 us). Needs G % 4 == 0 and U % 4 == 0.
template <int F, int P, int U, int W, int XM, int MG>
__global__ void __launch_bounds__(W * kWave) gemv_batch_kernel(BatchParams p)
{
    constexpr bool I4 = (F == kI4 || F == kI4ZP);
    constexpr int BKB = BatchFmt<F>::kBytesKB;
    constexpr int L = BatchFmt<F>::kLoads;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int lane = lane_id();
    const int wave = wave_id();
    const int ln = lane & 15;   // B column (weight row of the tile) and A row (activation row) of this lane
    const int lh = lane >> 4;   // k-group of this lane
    const int S = p.S;
    const int split = wave % S;
    const int tile0 = ((int)blockIdx.x * (W / S) + wave / S) * P;
    const int kb0 = split * p.kbs;
    const int nkb = max(0, min(p.KB, kb0 + p.kbs) - kb0);   // this wave's k-blocks
    const int M = p.M;
    const uint32_t c43 = (uint32_t)__builtin_amdgcn_readfirstlane(0x43434343);

    // Per-tile descriptors bounded to the tile's rows: rows >= N read zeros with no traffic. The row count goes
    // through readfirstlane: computed with v_med3 it would sit in a VGPR, and a descriptor built from a VGPR makes
    // the compiler wrap every load in a waterfall loop.
    __amdgpu_buffer_rsrc_t rw[P];
    __amdgpu_buffer_rsrc_t rm[I4 ? P : 1];
    __amdgpu_buffer_rsrc_t rz[F == kI4ZP ? P : 1];
#pragma unroll
    for (int t = 0; t < P; ++t) {
        const int row0 = (tile0 + t) * kTileRows;
        const uint32_t rows = (uint32_t)__builtin_amdgcn_readfirstlane(max(0, min(kTileRows, p.N - row0)));
        const size_t r0 = rows ? (size_t)row0 : 0;
        rw[t] = make_rsrc(p.W + r0 * p.row_bytes, rows * p.row_bytes);
        if constexpr (I4) rm[t] = make_rsrc((const uint8_t*)p.meta + r0 * p.meta_bytes, rows * p.meta_bytes);
        if constexpr (F == kI4ZP) rz[t] = make_rsrc(p.zeros + r0 * p.zbytes, rows * p.zbytes);
    }

    // Lane offsets. Weight: row ln of the tile, k-group lh. K tail (BF16/FP8, K % 128 != 0): load i of this lane
    // starts at column kb*128 + kcol[i] and is read only if that column is < K (K % 8 / K % 16 make each 16-byte load
    // all-in or all-out).
    const uint32_t lw = (uint32_t)ln * p.row_bytes + (uint32_t)lh * 16u;
    int klim[L];
#pragma unroll
    for (int i = 0; i < L; ++i) klim[i] = p.K - (F == kBF16 ? 32 * i + 8 * lh : 64 * i + 16 * lh);
    const uint32_t lmeta = (uint32_t)ln * p.meta_bytes;
    const uint32_t lzero = (uint32_t)ln * p.zbytes;

    // X=1: A-fragment offsets of this lane (row ln of x; rows >= M read zeros), step j adds a constant.
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(p.x, (uint32_t)M * (uint32_t)p.K * 2u);
    const bool xrow_ok = ln < M;
    const uint32_t lxa = ((uint32_t)ln * (uint32_t)p.K + (uint32_t)step_col<F>(0, lh)) * 2u;

    static_assert(MG == 1 || (I4 && U % 4 == 0), "grouped metadata needs INT4 and stages in fours");
    struct Stage {
        u32x4 w[P][L];
        uint32_t s[I4 ? P : 1][MG == 4 ? 2 : 1];   // MG=4: four 16-bit scales of groups kb..kb+3
        uint32_t z[F == kI4ZP ? P : 1];            // MG=4: four 4-bit zero points of groups kb..kb+3
        u32x4 a[XM ? 4 : 1];
    };
    // MG=4: the metadata of the current four groups, taken from the stage that loaded them
    uint32_t cur_s[I4 ? P : 1][2];
    uint32_t cur_z[F == kI4ZP ? P : 1];
    // Loads of this wave's k-block number t (t >= nkb: out of range, zeros, no traffic). Unconditional, so the
    // compiler never has to wait for the other stages' loads.
    auto issue = [&](Stage& B, int t, int u) {
        const bool ok = t < nkb;
        const int kb = kb0 + t;
        const uint32_t base = ok ? lw + (uint32_t)kb * (uint32_t)BKB : kOOB;
#pragma unroll
        for (int i = 0; i < L; ++i) {
            uint32_t off = base + (uint32_t)(64 * i);
            if constexpr (!I4) off = kb * kBlockCols < klim[i] ? off : kOOB;
#pragma unroll
            for (int tt = 0; tt < P; ++tt) B.w[tt][i] = ld16<PAIA_BATCH_WAUX>(rw[tt], off, 0u);
        }
        if constexpr (I4) {
            const uint32_t moff = ok ? lmeta + (uint32_t)kb * 2u : kOOB;
            const uint32_t zoff = ok ? lzero + (uint32_t)(kb >> 1) : kOOB;
            // MG=4: u is the unrolled stage slot, so this test folds away (no load under a runtime branch)
            if (MG == 1 || u % 4 == 0) {
#pragma unroll
                for (int tt = 0; tt < P; ++tt) {
                    if constexpr (MG == 4) {
                        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rm[tt], moff, 0u, 0);
                        B.s[tt][0] = v[0];
                        B.s[tt][1] = v[1];
                        if constexpr (F == kI4ZP) B.z[tt] = ld_u16(rz[tt], zoff, 0u);
                    } else {
                        B.s[tt][0] = ld_u16(rm[tt], moff, 0u);
                        if constexpr (F == kI4ZP) B.z[tt] = ld_u8(rz[tt], zoff, 0u);
                    }
                }
            }
        }
        if constexpr (XM) {
            const uint32_t xb = ok && xrow_ok ? lxa + (uint32_t)kb * 256u : kOOB;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t off = xb + (uint32_t)(2 * (step_col<F>(j, lh) - step_col<F>(0, lh)));
                if constexpr (!I4) off = kb * kBlockCols + step_col<F>(j, lh) < p.K ? off : kOOB;
                B.a[j] = ld16<0>(xrs, off, 0u);
            }
        }
    };

    // Epilogue operands (FP8 scale, bias) of row ln of each tile.
    uint32_t ep_scale[P], ep_bias[P];
    auto ep_load = [&]() {
#pragma unroll
        for (int t = 0; t < P; ++t) {
            const int row = (tile0 + t) * kTileRows + ln;
            const uint32_t off = row < p.N ? (uint32_t)row : (kOOB >> 2);
            ep_scale[t] = 0u;
            if constexpr (F == kFP8)
                ep_scale[t] = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(p.meta, (uint32_t)p.N * 4u), off * 4u, 0u, 0);
            ep_bias[t] = ld_u16(make_rsrc(p.bias ? p.bias : p.x, p.bias ? (uint32_t)p.N * 2u : 0u), off * 2u, 0u);
        }
    };

    // ---- X=0 x staging: chunk c holds, for every split s, k-blocks s*kbs + c*C .. +C-1 of all M rows, one 16-byte
    // vector (8 columns) per thread and step.
    const int nvec = XM ? 0 : S * M * p.C * 16;
    auto x_src = [&](int c, int q) -> uint32_t {
        const int v = q & 15;
        int r = q >> 4;
        const int kbl = r % p.C;
        r /= p.C;
        const int m = r % M, s2 = r / M;
        const int kbw = c * p.C + kbl;   // k-block within the split
        const int kg = s2 * p.kbs + kbw;
        const bool ok = kbw < p.kbs && kg < p.KB && kg * kBlockCols + 8 * v < p.K;
        return ok ? ((uint32_t)m * (uint32_t)p.K + (uint32_t)(kg * kBlockCols + 8 * v)) * 2u : kOOB;
    };
    auto x_put = [&](int q, u32x4 v) {
        const int vi = q & 15;
        int r = q >> 4;
        const int kbl = r % p.C;
        r /= p.C;
        const int m = r % M, s2 = r / M;
        if constexpr (I4) v = i4_pair_x(v);
        *reinterpret_cast<u32x4*>(smem + (uint32_t)(s2 * M + m) * p.xrow + (uint32_t)(kbl * 256 + vi * 16)) = v;
    };
    auto stage_x = [&](int c) {
        for (int q = (int)threadIdx.x; q < nvec; q += W * kWave) x_put(q, ld16<0>(xrs, x_src(c, q), 0u));
    };

    // X=0 A fragments: lane reads row (ln < M ? ln : 0) of its split's chunk.
    const uint32_t lx = XM ? 0u : (uint32_t)(split * M + (ln < M ? ln : 0)) * p.xrow + (uint32_t)(2 * step_col<F>(0, lh));
    // bf16 1.0 pairs: the B operand that turns an MFMA into row sums of A
    const uint32_t one2 = (uint32_t)__builtin_amdgcn_readfirstlane(0x3F803F80);
    const u32x4 ones = {one2, one2, one2, one2};

    f32x4 acc[P];
#pragma unroll
    for (int t = 0; t < P; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // k-block t of this wave (chunk-local index kbl, stage slot u).
    auto consume = [&](const Stage& B, int kbl, int t_idx, int u) {
        if constexpr (MG == 4) {
            if (u % 4 == 0) {
#pragma unroll
                for (int tt = 0; tt < P; ++tt) {
                    cur_s[tt][0] = B.s[tt][0];
                    cur_s[tt][1] = B.s[tt][1];
                    if constexpr (F == kI4ZP) cur_z[tt] = B.z[tt];
                }
            }
        }
        bf16x8 a[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (XM)
                a[j] = __builtin_bit_cast(bf16x8, I4 ? i4_pair_x(B.a[j]) : B.a[j]);
            else
                a[j] = *reinterpret_cast<const bf16x8*>(smem + lx + (uint32_t)kbl * 256u +
                                                        (uint32_t)(2 * (step_col<F>(j, lh) - step_col<F>(0, lh))));
        }
        // INT4: group sums of x for the D rows this lane holds (rows 4*lh + v), from an MFMA chain against ones
        f32x4 xs4 = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (I4) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xs4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j], __builtin_bit_cast(bf16x8, ones), xs4, 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < P; ++t) {
            if constexpr (F == kBF16) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j], __builtin_bit_cast(bf16x8, B.w[t][j]),
                                                                      acc[t], 0, 0, 0);
            } else if constexpr (F == kFP8) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const u32x4 w = B.w[t][j >> 1];
                    const uint32_t d0 = (j & 1) ? w.z : w.x, d1 = (j & 1) ? w.w : w.y;
                    const u32x4 b = {fp8x2_to_bf16x2<false>(d0), fp8x2_to_bf16x2<true>(d0), fp8x2_to_bf16x2<false>(d1),
                                     fp8x2_to_bf16x2<true>(d1)};
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j], __builtin_bit_cast(bf16x8, b), acc[t], 0, 0,
                                                                      0);
                }
            } else {
                f32x4 g = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const u32x4 w4 = B.w[t][0];
                    const uint32_t w = j == 0 ? w4.x : (j == 1 ? w4.y : (j == 2 ? w4.z : w4.w));
                    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
                    const u32x4 b = {__builtin_amdgcn_perm(c43, lo, 0x04010400u), __builtin_amdgcn_perm(c43, lo, 0x04030402u),
                                     __builtin_amdgcn_perm(c43, hi, 0x04010400u), __builtin_amdgcn_perm(c43, hi, 0x04030402u)};
                    g = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j], __builtin_bit_cast(bf16x8, b), g, 0, 0, 0);
                }
                float s, zc;
                uint32_t s16, z4;
                if constexpr (MG == 4) {
                    const int j = u % 4;   // group kb = chunk start + j
                    s16 = (cur_s[t][j >> 1] >> ((j & 1) * 16)) & 0xFFFFu;
                    z4 = F == kI4ZP ? (cur_z[t] >> (j * 4)) & 0xFu : 8u;
                } else {
                    const int kb = kb0 + t_idx;   // zero point of group kb: nibble kb & 1 of byte kb / 2
                    s16 = B.s[t][0];
                    z4 = F == kI4ZP ? (B.z[t] >> ((kb & 1) * 4)) & 0xFu : 8u;
                }
                if constexpr (F == kI4) {
                    s = f16_to_f32(s16);
                    zc = 136.0f;   // 128 (decode offset) + 8 (zero point)
                } else {
                    s = bf16_to_f32(s16);
                    zc = 128.0f + (float)z4;
                }
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(s, __builtin_fmaf(-zc, xs4[v], g[v]), acc[t][v]);
            }
        }
    };

    // First chunk (X=0): x loads go out first, then the first U k-blocks of weights, then x is stored (waiting on the
    // x loads only) while the weights are in flight. X=1 only issues the first U k-blocks.
    constexpr int XE = XM ? 1 : 2;
    u32x4 xe[XE];
    if constexpr (!XM) {
#pragma unroll
        for (int e = 0; e < XE; ++e) {
            const int q = (int)threadIdx.x + e * W * kWave;
            xe[e] = ld16<0>(xrs, q < nvec ? x_src(0, q) : kOOB, 0u);
        }
    }
    Stage buf[U];
#pragma unroll
    for (int u = 0; u < U; ++u) issue(buf[u], u, u);
    ep_load();
    if constexpr (!XM) {
#pragma unroll
        for (int e = 0; e < XE; ++e) {
            const int q = (int)threadIdx.x + e * W * kWave;
            if (q < nvec) x_put(q, xe[e]);
        }
        for (int q = (int)threadIdx.x + XE * W * kWave; q < nvec; q += W * kWave)
            x_put(q, ld16<0>(xrs, x_src(0, q), 0u));
        __syncthreads();
    }

    for (int c = 0; c < p.nchunks; ++c) {
        if (c > 0) {
            __syncthreads();
            stage_x(c);
            __syncthreads();
        }
        const int t_end = nkb - c * p.C;   // this wave's k-blocks left from this chunk on
        for (int kbl = 0; kbl < p.C; kbl += U) {
            if (kbl >= t_end) break;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int t = c * p.C + kbl + u;
                if (kbl + u < t_end) consume(buf[u], kbl + u, t, u);
                issue(buf[u], t + U, u);
            }
        }
    }

    // Split-K: splits 1..S-1 park their partials, split 0 adds them in split order and stores.
    if (S > 1) {
        __syncthreads();
        f32x4* part = reinterpret_cast<f32x4*>(smem);
        const int slot0 = (wave / S) * (S - 1);
        if (split > 0) {
#pragma unroll
            for (int t = 0; t < P; ++t) part[((slot0 + split - 1) * P + t) * kWave + lane] = acc[t];
        }
        __syncthreads();
        if (split > 0) return;
        for (int s2 = 1; s2 < S; ++s2)
#pragma unroll
            for (int t = 0; t < P; ++t) acc[t] += part[((slot0 + s2 - 1) * P + t) * kWave + lane];
    }

#pragma unroll
    for (int t = 0; t < P; ++t) {
        const int row = (tile0 + t) * kTileRows + ln;
        if (row >= p.N) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int m = 4 * lh + v;
            if (m < M) {
                float o = acc[t][v];
                if constexpr (F == kFP8) o = o * __uint_as_float(ep_scale[t]);
                if (p.bias) o = o + bf16_to_f32(ep_bias[t]);
                p.y[(size_t)m * (size_t)p.N + (size_t)row] = (uint16_t)f32_to_bf16_out(o);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------------------------------

// LDS a batch launch may use (bytes): the default budget, and the wider one of the X = 2 variants (x staged as for
// X = 0 in chunks of up to 80 KiB: two blocks still fit a 160 KiB CU, and fewer chunks mean fewer x reloads and
// barriers at M = 8..16).
constexpr uint32_t kBatchLds = 65536;
constexpr uint32_t kBatchLdsWide = 81920;

// Fill in the launch plan (k-blocks, splits, chunking, LDS) within `budget` bytes of LDS. Returns the LDS bytes
// (possibly 0 for X=1 without split-K), or -1 if no chunk of U k-blocks fits (X=0: too many activation rows x splits
// for this U).
template <int P, int U, int W, int XM, int MG>
int64_t batch_plan(BatchParams& p, uint32_t budget)
{
    p.KB = (p.K + kBlockCols - 1) / kBlockCols;
    p.ntiles = (p.N + kTileRows - 1) / kTileRows;
    p.kbs = (p.KB + p.S - 1) / p.S;
    if (MG == 4) p.kbs = (p.kbs + 3) / 4 * 4;   // every split starts on a four-group boundary
    const int cap = (p.kbs + U - 1) / U * U;
    const uint32_t pb = batch_part_bytes(p.S, W, P);
    if (XM) {
        p.C = cap;
        p.nchunks = 1;
        p.xrow = 0;
        return pb;
    }
    const uint32_t per_kb = batch_x_bytes(p.S, p.M, 1) - batch_x_bytes(p.S, p.M, 0);
    const uint32_t fixed = batch_x_bytes(p.S, p.M, 0);
    if (fixed + per_kb * U > budget) return -1;
    int C = (int)((budget - fixed) / per_kb);
    C -= C % U;
    if (C > cap) C = cap;
    p.C = C;
    p.nchunks = (p.kbs + C - 1) / C;
    p.xrow = (uint32_t)(C * 256 + 16);
    const uint32_t xb = batch_x_bytes(p.S, p.M, C);
    return xb > pb ? xb : pb;
}

// Launch on `st` with at most `budget` bytes of LDS. Arguments were validated by the caller (1 <= M <= 16, S divides
// W). Returns 0, -2 or a hipError_t.
template <int F, int P, int U, int W, int XM, int MG>
int launch_batch_mg(BatchParams p, hipStream_t st, uint32_t budget)
{
    const int64_t lds = batch_plan<P, U, W, XM, MG>(p, budget);
    if (lds < 0) return -2;
    if (lds > (int64_t)kBatchLds) {   // beyond the default dynamic-LDS limit: raise it once for this kernel
        static std::atomic<int> raised{0};
        if (!raised.load(std::memory_order_relaxed)) {
            const hipError_t e =
                hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_batch_kernel<F, P, U, W, XM, MG>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)budget);
            if (e != hipSuccess) return (int)e;
            raised.store(1, std::memory_order_relaxed);
        }
    }
    const int tiles_per_block = (W / p.S) * P;
    const int grid = (p.ntiles + tiles_per_block - 1) / tiles_per_block;
    hipLaunchKernelGGL((gemv_batch_kernel<F, P, U, W, XM, MG>), dim3(grid), dim3(W * kWave), (uint32_t)lds, st, p);
    return (int)hipGetLastError();
}

// INT4 with stages in fours and G % 4 == 0 (every Llama / Qwen shape) takes the grouped-metadata kernel.
template <int F, int P, int U, int W, int XM>
int launch_batch(BatchParams p, hipStream_t st, uint32_t budget = kBatchLds)
{
    if constexpr ((F == kI4 || F == kI4ZP) && U % 4 == 0) {
        if ((p.K / kBlockCols) % 4 == 0) return launch_batch_mg<F, P, U, W, XM, 4>(p, st, budget);
    }
    return launch_batch_mg<F, P, U, W, XM, 1>(p, st, budget);
}

using BatchLaunchFn = int (*)(BatchParams, hipStream_t);

struct BatchVariant {
    int P, U, W, S, X;
    BatchLaunchFn fn;
};

}  // namespace paia
