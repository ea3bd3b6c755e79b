// The fused M=1 GEMV kernel for gfx950, one template for all four weight formats.
//
//   y[n] = bf16_rn( sum_k deq(W[n,k]) * x[k]  (+ bias[n]) )
//
// Replaces the reference's per-format CUDA kernels (src/paia_gemv/gemv_bf16.cuh:97-134, gemv_fp8.cuh:84-113,
// gemv_int4.cuh:88-122) with a design for CDNA4:
//   * wave64: a wave reads one 1 KiB "chunk" of a weight row per 16-byte buffer load (64 lanes x 16 B); R rows per
//     wave share every x value they read.
//   * x is staged once per block into LDS, already converted to the pairing the format's dot product wants
//     (natural bf16 pairs for BF16/FP8; (k, k+4) pairs for INT4) plus, for INT4, the sum of each lane's 32 x values.
//   * weights are streamed with raw buffer loads bounded to the row: loads past K or past N return zeros, so the hot
//     loop has no per-lane predicates; two register buffers of R*U loads alternate so the next batch is in flight while
//     the current one is consumed.
//   * dequantisation happens in registers: FP8 via the gfx950 OCP e4m3->f32 convert packed to bf16, INT4 by masking nibbles into
//     the mantissa of bf16 128.0; every product is a v_dot2 bf16 with fp32 accumulation.
//   * the grid is persistent: ceil(tiles / T) blocks each take T tiles (T chosen so the grid fits the resident-block
//     capacity of the device), which keeps the per-block x staging amortised and the load balanced.
//   * KSPLIT (variant knob H=1): the W waves of a block share R rows and split the row's chunks round-robin; partial
//     sums meet in LDS (fixed order, so results are reproducible). This is the split-K used for tall-K shapes.
//
// No MFMA: at M=1 the arithmetic intensity is ~1-4 FLOP/byte and the kernel is HBM-bound.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "gemv_device.h"

namespace paia {

struct GemvParams {
    const uint8_t* W;       // weight rows, row_bytes each
    const void* meta;       // FP8: fp32 scale [N]; INT4: fp16 scale [N][G]; INT4ZP: bf16 scale [N][G]
    const uint8_t* zeros;   // INT4ZP: [N][zbytes] packed 4-bit zero points
    const uint16_t* x;      // bf16 [K]
    const uint16_t* bias;   // bf16 [N] or null
    uint16_t* y;            // bf16 [N]
    int N, K;
    uint32_t row_bytes;     // weight bytes per row
    uint32_t meta_bytes;    // INT4: scale bytes per row (2 G)
    uint32_t zbytes;        // INT4ZP: zero-point bytes per row (ceil(G/2))
    int nchunks;            // ceil(row_bytes / 1 KiB)
    int tiles;              // row tiles
};

// LDS footprint of a launch (bytes): staged x, INT4 segment sums, split-K partials.
template <int F>
__host__ __device__ constexpr uint32_t lds_x_bytes(int nchunks)
{
    return (uint32_t)nchunks * FmtInfo<F>::kXQ * kChunkBytes;
}
template <int F>
__host__ __device__ constexpr uint32_t lds_s32_bytes(int nchunks)
{
    return (F == kI4 || F == kI4ZP) ? (uint32_t)nchunks * kWave * 4u : 0u;
}

// Stage x (bf16, K values) into LDS as nchunks * XQ * 64 16-byte vectors. Vector (c, j, lane) sits at index
// (c*XQ + j)*64 + lane and holds columns c*CC + lane*CPL + 8j .. +7, where CPL = 8*XQ columns per lane and
// CC = 64*CPL columns per chunk: a lane's x for chunk c is XQ conflict-free ds_read_b128s. Columns >= K are zero.
template <int F>
__device__ __forceinline__ void stage_x(const GemvParams& p, u32x4* xs, float* s32)
{
    constexpr int XQ = FmtInfo<F>::kXQ;
    const int nq = p.nchunks * XQ * kWave;
    for (int q = (int)threadIdx.x; q < nq; q += (int)blockDim.x) {
        const int c = q / (XQ * kWave), r = q - c * (XQ * kWave);
        const int l = r / XQ, j = r - l * XQ;
        const int col = q * 8;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (col < p.K) v = *reinterpret_cast<const u32x4*>(p.x + col);
        if constexpr (F == kI4 || F == kI4ZP) {
            // segment sum of this vector's 8 values (fixed order), then over the quad = the lane's 32 columns
            float s8 = ((bf16_to_f32(v.x & 0xFFFFu) + bf16_to_f32(v.x >> 16)) +
                        (bf16_to_f32(v.y & 0xFFFFu) + bf16_to_f32(v.y >> 16))) +
                       ((bf16_to_f32(v.z & 0xFFFFu) + bf16_to_f32(v.z >> 16)) +
                        (bf16_to_f32(v.w & 0xFFFFu) + bf16_to_f32(v.w >> 16)));
            s8 = quad_sum(s8);   // nq and blockDim are multiples of 4: quads are fully active together
            if (j == 0) s32[c * kWave + l] = s8;
            // pair (x0,x4),(x1,x5),(x2,x6),(x3,x7) to match the nibble order of i4_word_dot
            const u32x4 a = v;
            v.x = (a.x & 0xFFFFu) | (a.z << 16);
            v.y = (a.x >> 16) | (a.z & 0xFFFF0000u);
            v.z = (a.y & 0xFFFFu) | (a.w << 16);
            v.w = (a.y >> 16) | (a.w & 0xFFFF0000u);
        }
        xs[(c * XQ + j) * kWave + l] = v;
    }
}

template <int F, int R, int U>
struct WBuf {
    u32x4 w[R][U];
    uint32_t s[(F == kI4 || F == kI4ZP) ? R : 1][(F == kI4 || F == kI4ZP) ? U : 1];
    uint32_t z[F == kI4ZP ? R : 1][F == kI4ZP ? U : 1];
};

template <int F, int R, int U, int W, int AUX, bool KSPLIT>
__global__ void __launch_bounds__(W * kWave) gemv_kernel(GemvParams p)
{
    constexpr int XQ = FmtInfo<F>::kXQ;
    constexpr bool I4 = (F == kI4 || F == kI4ZP);
    constexpr int ROWS_PER_TILE = KSPLIT ? R : R * W;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    u32x4* xs = reinterpret_cast<u32x4*>(smem);
    float* s32 = reinterpret_cast<float*>(smem + lds_x_bytes<F>(p.nchunks));
    float* part = reinterpret_cast<float*>(smem + lds_x_bytes<F>(p.nchunks) + lds_s32_bytes<F>(p.nchunks));

    const int lane = lane_id();
    const int wave = wave_id();
    const int nchunks = p.nchunks;

    stage_x<F>(p, xs, s32);
    __syncthreads();

    // chunks handled by this wave in each tile, and batches of U of them
    const int my_chunks = KSPLIT ? (nchunks > wave ? (nchunks - wave + W - 1) / W : 0) : nchunks;
    const int nb = (my_chunks + U - 1) / U;
    const uint32_t voff16 = (uint32_t)lane * 16u;

    int it = 0;
    for (int tile = (int)blockIdx.x; tile < p.tiles; tile += (int)gridDim.x, ++it) {
        const int row0 = tile * ROWS_PER_TILE + (KSPLIT ? 0 : wave * R);
        __amdgpu_buffer_rsrc_t wr[R];
        __amdgpu_buffer_rsrc_t mr[I4 ? R : 1];
        __amdgpu_buffer_rsrc_t zr[F == kI4ZP ? R : 1];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = row0 + r;
            const bool ok = row < p.N;
            const size_t rr = ok ? (size_t)row : 0;
            wr[r] = make_rsrc(p.W + rr * p.row_bytes, ok ? p.row_bytes : 0u);
            if constexpr (I4) mr[r] = make_rsrc((const uint8_t*)p.meta + rr * p.meta_bytes, ok ? p.meta_bytes : 0u);
            if constexpr (F == kI4ZP) zr[r] = make_rsrc(p.zeros + rr * p.zbytes, ok ? p.zbytes : 0u);
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;

        auto chunk_of = [&](int b, int u) { return KSPLIT ? wave + W * (b * U + u) : b * U + u; };

        // Loads are issued unconditionally: a chunk past the row end reads as zeros through the bounded descriptor
        // (no memory traffic). The whole offset goes in the per-lane voffset (soffset = 0), the operand the
        // descriptor's range check covers. Keeping the issue branch-free lets the compiler wait for exactly the batch being
        // consumed (s_waitcnt vmcnt(#loads of the other batch)) instead of draining both buffers.
        auto issue = [&](WBuf<F, R, U>& B, int b) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t c = (uint32_t)chunk_of(b, u);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    B.w[r][u] = ld16<AUX>(wr[r], voff16 + c * kChunkBytes, 0u);
                    if constexpr (I4) B.s[r][u] = ld_u16(mr[r], (uint32_t)(lane >> 2) * 2u + c * 32u, 0u);
                    if constexpr (F == kI4ZP) B.z[r][u] = ld_u8(zr[r], (uint32_t)(lane >> 3) + c * 8u, 0u);
                }
            }
        };

        // Chunks past the row end hold zero weights (and zero INT4 scales); their x index is clamped to the last
        // staged chunk so every product stays 0 * finite.
        auto consume = [&](const WBuf<F, R, U>& B, int b) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                int c = chunk_of(b, u);
                c = c < nchunks ? c : nchunks - 1;
                u32x4 xv[XQ];
#pragma unroll
                for (int j = 0; j < XQ; ++j) xv[j] = xs[(c * XQ + j) * kWave + lane];
                if constexpr (F == kBF16) {
#pragma unroll
                    for (int r = 0; r < R; ++r) acc[r] = dot_bf16_16B(B.w[r][u], xv[0], acc[r]);
                } else if constexpr (F == kFP8) {
#pragma unroll
                    for (int r = 0; r < R; ++r) acc[r] = dot_fp8_16B(B.w[r][u], xv[0], xv[1], acc[r]);
                } else {
                    const float sx = s32[c * kWave + lane];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const float d = dot_i4_16B(B.w[r][u], xv[0], xv[1], xv[2], xv[3]);
                        float s, zc;
                        if constexpr (F == kI4) {
                            s = f16_to_f32(B.s[r][u]);
                            zc = 136.0f;                              // 128 (magic) + 8 (zero point)
                        } else {
                            s = bf16_to_f32(B.s[r][u]);
                            const uint32_t z = (B.z[r][u] >> (((uint32_t)lane >> 2) & 1u) * 4u) & 0xFu;
                            zc = 128.0f + (float)z;
                        }
                        acc[r] = __builtin_fmaf(s, __builtin_fmaf(-zc, sx, d), acc[r]);
                    }
                }
            }
        };

        WBuf<F, R, U> A, B;
        if (nb > 0) {
            issue(A, 0);
            for (int b = 0;; b += 2) {
                issue(B, b + 1);
                consume(A, b);
                if (b + 1 >= nb) break;
                issue(A, b + 2);
                consume(B, b + 1);
                if (b + 2 >= nb) break;
            }
        }

        // reduce each row over the wave, then (split-K) over the block's waves
        float tot[R];
#pragma unroll
        for (int r = 0; r < R; ++r) tot[r] = wave_sum(acc[r]);

        auto store_row = [&](int row, float v) {
            if (row >= p.N) return;
            if constexpr (F == kFP8) v = v * reinterpret_cast<const float*>(p.meta)[row];
            if (p.bias) v = v + bf16_to_f32(p.bias[row]);
            p.y[row] = (uint16_t)f32_to_bf16_rne(v);
        };

        if constexpr (!KSPLIT) {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r) store_row(row0 + r, tot[r]);
            }
        } else {
            float* slot = part + (it & 1) * (W * R);
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r) slot[wave * R + r] = tot[r];
            }
            __syncthreads();
            if (wave == 0 && lane < R) {
                float v = 0.0f;
#pragma unroll
                for (int w = 0; w < W; ++w) v += slot[w * R + lane];
                store_row(row0 + lane, v);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------------------------------

// Device facts used to size the persistent grid (queried once; the library assumes one GPU model per process).
struct DeviceFacts {
    int cus = 0;
    int lds_per_cu = 0;
};
DeviceFacts device_facts();

// Largest LDS a launch may request (bytes). Beyond it the entry points return -2.
constexpr uint32_t kMaxLds = 65536;

template <int F, int R, int U, int W, int AUX, bool KSPLIT>
uint32_t gemv_lds_bytes(int nchunks)
{
    return lds_x_bytes<F>(nchunks) + lds_s32_bytes<F>(nchunks) + (KSPLIT ? 2u * W * R * 4u : 0u);
}

template <int F, int R, int U, int W, int AUX, bool KSPLIT>
int gemv_max_blocks_per_cu()
{
    static std::atomic<int> cached{0};
    int v = cached.load(std::memory_order_relaxed);
    if (v == 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_kernel<F, R, U, W, AUX, KSPLIT>, W * kWave, 0) !=
                hipSuccess || n <= 0)
            n = 1;
        cached.store(n, std::memory_order_relaxed);
        v = n;
    }
    return v;
}

// Launch on `st`. Arguments were validated by the caller. Returns 0, -2 (LDS limit), or a hipError_t.
template <int F, int R, int U, int W, int AUX, bool KSPLIT>
int launch_gemv(GemvParams p, hipStream_t st)
{
    p.nchunks = (int)((p.row_bytes + kChunkBytes - 1) / kChunkBytes);
    const int rows_per_tile = KSPLIT ? R : R * W;
    p.tiles = (p.N + rows_per_tile - 1) / rows_per_tile;
    const uint32_t lds = gemv_lds_bytes<F, R, U, W, AUX, KSPLIT>(p.nchunks);
    if (lds > kMaxLds) return -2;
    const DeviceFacts df = device_facts();
    int per_cu = gemv_max_blocks_per_cu<F, R, U, W, AUX, KSPLIT>();
    if (df.lds_per_cu > 0) {
        const int by_lds = (int)(df.lds_per_cu / (lds ? lds : 1u));
        if (by_lds < per_cu) per_cu = by_lds > 0 ? by_lds : 1;
    }
    const int gmax = (df.cus > 0 ? df.cus : 256) * per_cu;
    int grid = p.tiles < gmax ? p.tiles : gmax;
    const int per_block = (p.tiles + grid - 1) / grid;
    grid = (p.tiles + per_block - 1) / per_block;
    hipLaunchKernelGGL((gemv_kernel<F, R, U, W, AUX, KSPLIT>), dim3(grid), dim3(W * kWave), lds, st, p);
    return (int)hipGetLastError();
}

using GemvLaunchFn = int (*)(GemvParams, hipStream_t);

struct Variant {
    int R, U, W, S, H;
    GemvLaunchFn fn;
};

inline bool aligned(const void* ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0; }

}  // namespace paia
