// The fused M=1 GEMV kernel for gfx950, one template for all four weight formats.
//
//   y[n] = bf16_rn( sum_k deq(W[n,k]) * x[k]  (+ bias[n]) )
//
// Replaces the reference's per-format CUDA kernels (src/paia_gemv/gemv_bf16.cuh:97-134, gemv_fp8.cuh:84-113,
// gemv_int4.cuh:88-122) with a design for CDNA4:
//   * Work unit ("item"): R consecutive rows x one K-segment of U 1-KiB chunks. A wave reads a chunk of a row with one
//     16-byte buffer load per lane (64 lanes x 16 B = 1 KiB), so an item is R*U loads.
//   * Each wave walks its own sequence of items and keeps the next item's loads in flight while it consumes the
//     current one (two register buffers, both filled while x is staged). There is no block-wide synchronisation in
//     the streaming loop, so the memory pipeline never drains at row-group boundaries.
//   * H=0: a wave owns whole row groups (all segments of a group are consecutive items of one wave; the partial sums
//     stay in registers). Groups are dealt to the waves of the grid round-robin, so at any moment the grid streams a
//     window of neighbouring rows.
//     H=1 (split-K): the W waves of a block share each of the block's row groups and take its segments round-robin;
//     per-wave partial sums go to LDS and are combined in a fixed order after a block barrier (one barrier per round
//     of up to `round` groups, not per group). This is the split-K used for tall-K / small-N shapes.
//   * x is staged once per block into LDS, already in the pairing each format's dot product wants (natural bf16
//     pairs for BF16/FP8; (k, k+4) pairs scaled by 2^64 / 2^60 for INT4) plus, for INT4, the sum of each lane's 32
//     x values. The first two items' weight loads are issued before the staging, so their latency overlaps it.
//   * Weight rows are read with raw buffer loads through one descriptor per row group; a lane whose 16 bytes lie past
//     the row end (K tails, padding segments, rows >= N) gets an out-of-range offset and reads zeros without a branch
//     or any memory traffic.
//   * Dequantisation happens in registers: FP8 via the gfx950 OCP e4m3 -> f32 convert packed to bf16, INT4 by
//     masking nibbles in place as bf16 subnormals (q * 2^-133, against x scaled by 2^64; the x-from-global kernel
//     masks them into the mantissa of bf16 128.0 instead); every product is a v_dot2 bf16 with fp32 accumulation.
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
    int nseg;               // ceil(nchunks / U): K-segments per row
    int ngroups;            // ceil(N / R): row groups
    int round;              // H=1: row groups per LDS round
};

// Out-of-range buffer offset: above any descriptor's num_records, so the load returns zeros.
constexpr uint32_t kOOB = 0x80000000u;

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
// INT4 staged x: per activation row 16 bytes of per-wave window flags and one u32 slot per wave for the largest |x|
// each wave saw (read only when the first scale does not stand), rounded to 16 bytes.
__host__ __device__ constexpr uint32_t lds_slot_bytes(int F, int MB, int W)
{
    return (F == kI4 || F == kI4ZP) ? (((uint32_t)MB * 16u + (uint32_t)(MB * W) * 4u + 15u) & ~15u) : 0u;
}

// x (bf16, K values) is staged into LDS as nchunks * XQ * 64 16-byte vectors. Vector q holds x[8q .. 8q+7] (zero
// past K) and sits at LDS index (c*XQ + j)*64 + l, where c = q / (XQ*64), l = (q mod XQ*64) / XQ, j = q mod XQ: lane
// l's x for chunk c (columns c*CC + l*CPL .. +CPL-1, CPL = 8*XQ columns per lane, CC = 64*CPL per chunk) is XQ
// conflict-free ds_read_b128s.
//
// Staging is split in two so the x loads go to memory ahead of the weight loads: x_load issues the block's first
// XE vectors per thread (buffer loads bounded to K: zeros past K; INT4 skips them), the caller then issues its first
// weight loads, and x_store writes them to LDS, waiting only for the x loads. Vectors beyond XE per thread (large K)
// are loaded and stored afterwards.
template <int XE>
struct XRegs {
    u32x4 v[XE];
};

// NT: threads per block (a compile-time constant, so no work-group size read from the dispatch packet).
template <int F, int XE, int NT>
__device__ __forceinline__ void x_load(const uint16_t* x, int K, XRegs<XE>& xr)
{
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)K * 2u);
#pragma unroll
    for (int e = 0; e < XE; ++e) {
        // INT4: only the vectors some thread of the block needs (x holds K*2 bytes), since a load past them is still
        // a vector-memory instruction for the CU to issue (measured on MI355X: INT4 o 4096x4096 3.87 -> 3.81 us,
        // reference format 3.80 -> 3.67, down 7.16 -> 7.11). BF16 and FP8 issue every load: the branch moved their
        // first waits in the loop earlier and was slower (FP8 o 4.78 -> 4.97, gate_up 18.82 -> 19.11).
        if constexpr (F == kI4 || F == kI4ZP) {
            xr.v[e] = u32x4{0u, 0u, 0u, 0u};
            if ((uint32_t)(e * NT) * 16u < (uint32_t)K * 2u)
                xr.v[e] = ld16<0>(xrs, ((uint32_t)threadIdx.x + (uint32_t)(e * NT)) * 16u, 0u);
        } else {
            xr.v[e] = ld16<0>(xrs, ((uint32_t)threadIdx.x + (uint32_t)(e * NT)) * 16u, 0u);
        }
    }
}

// INT4, x read from global memory (the x-from-global kernel): the sum of one x vector's 8 values (fixed order), and
// the vector re-paired (x0,x2),(x4,x6),(x1,x3),(x5,x7) to match the nibble order of i4_word_dot.
__device__ __forceinline__ float i4_pair_sum_x(u32x4& v)
{
    const float s8 = ((bf16_to_f32(v.x & 0xFFFFu) + bf16_to_f32(v.x >> 16)) +
                      (bf16_to_f32(v.y & 0xFFFFu) + bf16_to_f32(v.y >> 16))) +
                     ((bf16_to_f32(v.z & 0xFFFFu) + bf16_to_f32(v.z >> 16)) +
                      (bf16_to_f32(v.w & 0xFFFFu) + bf16_to_f32(v.w >> 16)));
    const u32x4 a = v;
    v.x = (a.x & 0xFFFFu) | (a.y << 16);
    v.y = (a.z & 0xFFFFu) | (a.w << 16);
    v.z = (a.x >> 16) | (a.y & 0xFFFF0000u);
    v.w = (a.z >> 16) | (a.w & 0xFFFF0000u);
    return s8;
}

// Constants of the INT4 staging: the lane sums' decode of q = 1 (i4_staged_sum) and the operands of
// i4_scale_pair_first (packed ones, and the first scale's exponent increments 64 and 60 in the bf16 exponent field).
// The last three pass through an empty asm statement (no instruction) so the compiler cannot see their values and
// keeps the packed minimum and multiply-add packed.
struct I4SumConsts {
    uint32_t c1, c16, one16, e64, e60;
    __device__ __forceinline__ I4SumConsts()
        : c1(0x00010001u), c16(0x00100010u), one16(0x00010001u), e64(0x20002000u), e60(0x1E001E00u)
    {
        asm("" : "+v"(one16), "+v"(e64), "+v"(e60));
    }
};
// The sum of an unscaled staged vector's 8 values (the 0x43-exponent decode's lane sums), by v_dot2 against (1, 1).
__device__ __forceinline__ float i4_unscaled_sum(const u32x4 sx)
{
    float s = dot2_bf16(sx.x, 0x3F803F80u, 0.0f);
    s = dot2_bf16(sx.y, 0x3F803F80u, s);
    s = dot2_bf16(sx.z, 0x3F803F80u, s);
    return dot2_bf16(sx.w, 0x3F803F80u, s);
}

// How x is staged for the INT4 kernels: for the subnormal decode at the first scale (integer operations) or at a
// picked scale (through fp32), or unscaled for the 0x43-exponent decode.
enum I4StageMode : int { kStageFirst = 0, kStageExact = 1, kStage43 = 2 };

// INT4, staged x for the subnormal decode (i4_word_decode_dn): the vector re-paired (x0,x4),(x1,x5),(x2,x6),(x3,x7)
// with pairs 0 and 2 scaled by 2^a and pairs 1 and 3 by 2^(a-4). kStageFirst: a = 64 with integer operations
// (i4_scale_pair_first), the |x| patterns folded into amax; kStageExact: exactly by 2^a through fp32; kStage43: only
// re-paired, unscaled.
template <int MODE>
__device__ __forceinline__ u32x4 i4_stage_x(const u32x4 v, int a, u16x2& amax, const I4SumConsts& k)
{
    if constexpr (MODE == kStage43) {
        // (x0,x2),(x4,x6),(x1,x3),(x5,x7), the nibble order of i4_word_dot
        return {__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x05040100u),
                __builtin_amdgcn_perm(v.y, v.x, 0x07060302u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)};
    }
    const u32x4 p = i4_pairs(v);
    if constexpr (MODE == kStageFirst) {
        static_assert(kI4StageFirst.a == 64, "the integer staging adds the first scale's exponents");
        return {i4_scale_pair_first(p.x, amax, k.one16, k.e64), i4_scale_pair_first(p.y, amax, k.one16, k.e60),
                i4_scale_pair_first(p.z, amax, k.one16, k.e64), i4_scale_pair_first(p.w, amax, k.one16, k.e60)};
    } else {
        return {i4_scale_pair_exact(p.x, a), i4_scale_pair_exact(p.y, a - 4), i4_scale_pair_exact(p.z, a),
                i4_scale_pair_exact(p.w, a - 4)};
    }
}

template <int F, int MODE = kStageFirst>
__device__ __forceinline__ void x_put(int q, u32x4 v, u32x4* xs, float* s32, int a, u16x2& amax,
                                      const I4SumConsts& k)
{
    constexpr int XQ = FmtInfo<F>::kXQ;
    const int c = q / (XQ * kWave), r = q - c * (XQ * kWave);
    const int l = r / XQ, j = r - l * XQ;
    if constexpr (F == kI4 || F == kI4ZP) {
        // the 4 vectors of a lane-segment are 4 consecutive q in one quad of threads: the quad sum is the lane's
        // 32-column x sum, in the decode's units (2^(a-133) for the subnormal decode, 1 for the 0x43 decode)
        v = i4_stage_x<MODE>(v, a, amax, k);
        const float s8 = quad_sum(MODE == kStage43 ? i4_unscaled_sum(v) : i4_staged_sum(v, k.c1, k.c16));
        if (j == 0) s32[c * kWave + l] = s8;
    }
    xs[(c * XQ + j) * kWave + l] = v;
}

// Store the XE early vectors, then load+store the rest. nq and NT are multiples of 4, so the `q < nq` tests are
// uniform over each quad (quad_sum needs the whole quad). INT4: staged at the first scale (MODE kStageFirst: returns
// the largest sign-cleared bf16 pattern of the vectors this thread staged, their |x| maximum; vectors past K are
// zero) or unscaled (kStage43).
template <int F, int XE, int NT, int MODE = kStageFirst>
__device__ __forceinline__ uint32_t x_store(const uint16_t* x, int K, int nchunks, const XRegs<XE>& xr, u32x4* xs,
                                            float* s32)
{
    constexpr int XQ = FmtInfo<F>::kXQ;
    const int nq = nchunks * XQ * kWave;
    constexpr int T = NT;
    const I4SumConsts k;
    u16x2 amax = {0, 0};
#pragma unroll
    for (int e = 0; e < XE; ++e) {
        const int q = (int)threadIdx.x + e * T;
        if (q < nq) x_put<F, MODE>(q, xr.v[e], xs, s32, kI4StageFirst.a, amax, k);
    }
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)K * 2u);
    for (int q = (int)threadIdx.x + XE * T; q < nq; q += T)
        x_put<F, MODE>(q, ld16<0>(xrs, (uint32_t)q * 16u, 0u), xs, s32, kI4StageFirst.a, amax, k);
    return amax.x > amax.y ? amax.x : amax.y;
}

// INT4: stage the whole row again at the scale 2^a (every vector loaded from global memory again).
template <int F, int NT>
__device__ __forceinline__ void x_restage(const uint16_t* x, int K, int nchunks, u32x4* xs, float* s32, int a)
{
    const int nq = nchunks * FmtInfo<F>::kXQ * kWave;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)K * 2u);
    const I4SumConsts k;
    u16x2 unused = {0, 0};
    for (int q = (int)threadIdx.x; q < nq; q += NT)
        x_put<F, kStageExact>(q, ld16<0>(xrs, (uint32_t)q * 16u, 0u), xs, s32, a, unused, k);
}

// INT4 first-scale window flags of one wave (one byte per wave and activation row): bit 0 some |x| >= 2^-20, bit 1
// some |x| >= 2^64, bit 2 some x != 0. The first scale stands for the row when no wave set bit 1 and some wave set
// bit 0, or no wave set bit 2 (all zero: every scale gives zeros).
__device__ __forceinline__ uint32_t i4_window_flags(uint32_t tmax)
{
    return (__builtin_amdgcn_ballot_w64(tmax >= kI4FirstLoBits) != 0 ? 1u : 0u) |
           (__builtin_amdgcn_ballot_w64(tmax >= kI4FirstHiBits) != 0 ? 2u : 0u) |
           (__builtin_amdgcn_ballot_w64(tmax != 0u) != 0 ? 4u : 0u);
}
__device__ __forceinline__ bool i4_first_stands(uint32_t f_or)
{
    return (f_or & 0x02020202u) == 0u && ((f_or & 0x01010101u) != 0u || (f_or & 0x04040404u) == 0u);
}
// The OR of the W flag bytes at p (4-byte aligned), folded into the bytes of one word (the tests above look at every
// byte).
template <int W>
__device__ __forceinline__ uint32_t or_flag_bytes(const uint8_t* p)
{
    static_assert(W >= 1 && W <= 16, "waves per block");
    if constexpr (W != 4 && W != 8 && W != 16) {
        uint32_t f = 0u;
#pragma unroll
        for (int w = 0; w < W; ++w) f |= (uint32_t)p[w];
        return f;
    } else if constexpr (W == 4) {
        return *reinterpret_cast<const uint32_t*>(p);
    } else if constexpr (W == 8) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        return v.x | v.y;
    } else {
        const u32x4 v = *reinterpret_cast<const u32x4*>(p);
        return (v.x | v.y) | (v.z | v.w);
    }
}

// One item's registers: R*U weight loads, INT4 scales/zeros, (XG) the lane's x vectors of its U chunks, and the
// (wave-uniform) position of the item.
template <int F, int R, int U, bool XG = false>
struct Item {
    u32x4 w[R][U];
    u32x4 xg[XG ? U : 1][XG ? FmtInfo<F>::kXQ : 1];
    uint32_t s[(F == kI4 || F == kI4ZP) ? R : 1][(F == kI4 || F == kI4ZP) ? U : 1];
    uint32_t z[F == kI4ZP ? R : 1][F == kI4ZP ? U : 1];
    int group;           // row group (-1: no item)
    int chunk0;          // first chunk of the segment
    int k;               // index of the group in this wave's (H=0) or block's (H=1) sequence
    bool last;           // last item of its group for this wave
};

// Item buffers in flight per wave. Two: measured on MI355X, deeper pipelines of small items (8 x 1 KiB, 4 x 2 KiB)
// were slower than two buffers of larger items (2 x 4 KiB) at the same bytes in flight, because every item pays
// its issue/offset/epilogue bookkeeping; the bytes in flight are set by the item size R*U instead.
#ifndef PAIA_GEMV_PIPE_DEPTH
#define PAIA_GEMV_PIPE_DEPTH 2
#endif
template <int R, int U>
__host__ __device__ constexpr int pipe_depth()
{
    return PAIA_GEMV_PIPE_DEPTH;
}

// Walks a wave's items in order. H=0: groups g = first + k*gstride (k = 0..), every segment of each in turn.
// H=1: groups of the block g = blockIdx + k*gridDim, segments s = wave, wave+W, ... of each.
struct ItemWalker {
    int g0;            // first group of the sequence
    int g, s;          // next item
    int gstride, s0, sstep, nseg, ngroups;
    int k;             // index of the group within this block's / wave's sequence
    __device__ __forceinline__ bool valid() const { return g < ngroups && s0 < nseg; }
    __device__ __forceinline__ void advance()
    {
        s += sstep;
        if (s >= nseg) {
            s = s0;
            g += gstride;
            ++k;
        }
    }
};

// The kernel body. MB activation rows (x [MB][K], y [MB][N]): MB = 1 is the M = 1 GEMV (gemv_kernel); MB = 2..6 (BF16, FP8:
// 2..8) is the row-streaming small-batch kernel (gemv_rows_kernel): the same weight stream and decode, with MB
// accumulators per row and MB staged copies of x, so each weight is loaded and decoded once for all activation rows.
// XG: x is not staged; each item's loads bring the lane's x vectors from global memory (L2) with the weights. For K
// whose staged x would not fit the LDS (M = 1 only).
// D43 (INT4, M = 1, staged x): the 0x43-exponent decode against unscaled staged x, for launches whose waves make
// few weight loads (launch_gemv chooses); otherwise staged INT4 x feeds the subnormal decode.
// DR (M = 1, H = 0): the walk ends in a drain, for launches whose waves take at most two items (launch_gemv chooses).
template <int F, int R, int U, int W, int AUX, bool KSPLIT, int MB, bool XG = false, bool D43 = false, bool DR = false>
__device__ __forceinline__ void gemv_body(const GemvParams& p)
{
    static_assert(MB >= 1 && MB <= 8 && (MB <= 6 || F == kBF16 || F == kFP8) && (MB == 1 || !KSPLIT),
                  "activation rows: 1..6 (BF16, FP8 1..8), split-K only at M = 1");
    static_assert(!XG || MB == 1, "x from global memory: M = 1 only");
    constexpr int XQ = FmtInfo<F>::kXQ;
    constexpr bool I4 = (F == kI4 || F == kI4ZP);
    static_assert(!D43 || (I4 && !XG && MB == 1), "the unscaled staged INT4 decode: M = 1 GEMV only");
    static_assert(!DR || (!KSPLIT && MB == 1), "the drain: row-parallel M = 1 launches only");
    constexpr bool DN = I4 && !XG && !D43;   // the subnormal decode against x staged at a power-of-two scale
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    // LDS: MB staged copies of x, then MB copies of the INT4 lane sums, the INT4 per-wave |x| maxima, then (H=1) the
    // split-K partials
    const uint32_t xrow = XG ? 0u : lds_x_bytes<F>(p.nchunks), srow = XG ? 0u : lds_s32_bytes<F>(p.nchunks);
    constexpr uint32_t slot_bytes = DN ? lds_slot_bytes(F, MB, W) : 0u;
    u32x4* xs = reinterpret_cast<u32x4*>(smem);
    float* s32 = reinterpret_cast<float*>(smem + MB * xrow);
    uint32_t* slots = reinterpret_cast<uint32_t*>(smem + MB * xrow + MB * srow);
    uint8_t* flags = reinterpret_cast<uint8_t*>(slots);   // INT4: [MB][16] per-wave window flags
    uint32_t* maxima = slots + 4 * MB;                     // INT4: [MB][W] per-wave largest |x| (second walk only)
    float* part = reinterpret_cast<float*>(smem + MB * xrow + MB * srow + slot_bytes);

    const int lane = lane_id();
    const int wave = wave_id();
    const uint32_t lane16 = (uint32_t)lane * 16u;
    const uint32_t gl = (uint32_t)lane >> 2;   // INT4: the lane's 32 weights lie in group gl of the chunk
    // INT4 decode constant, made opaque so it stays in one register instead of a literal per instruction
    const uint32_t c43 = (uint32_t)__builtin_amdgcn_readfirstlane(0x43434343);
    const uint32_t row_bytes = p.row_bytes;
    const int nchunks = p.nchunks;

    ItemWalker it;
    it.nseg = p.nseg;
    it.ngroups = p.ngroups;
    it.k = 0;
    if constexpr (!KSPLIT) {
        int lb = (int)blockIdx.x;
        if constexpr (DR) {
            // The drain kernels take their row groups through a logical block index that gives each of the 8 XCDs
            // (workgroups are dealt to them round-robin) a contiguous range of blocks, so a 128-byte line of the
            // outputs, row scales or bias is fetched and written by one XCD's L2 rather than by several (a bijection
            // for any grid). Measured on MI355X: FP8 qkv 6144x4096 6.02 -> 5.73 us, Qwen qkv + bias 4.96 -> 4.80, o
            // 4.79 -> 4.70, BF16 Qwen qkv + bias 7.05 -> 6.80; the INT4 launches within +-0.07. On launches with
            // more items per wave the same remap was slower (FP8 gate_up 18.90 -> 19.69), so only these take it.
            const int G = (int)gridDim.x, x = lb % 8, per = G / 8, rem = G % 8;
            lb = (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + lb / 8;
        }
        it.g = lb * W + wave;
        it.gstride = (int)gridDim.x * W;
        it.s0 = 0;
        it.sstep = 1;
    } else {
        it.g = (int)blockIdx.x;
        it.gstride = (int)gridDim.x;
        it.s0 = wave;
        it.sstep = W;
    }
    it.s = it.s0;
    it.g0 = it.g;

    // Per-row buffer descriptors of the current row group (wave-uniform, rebuilt only when the group changes). Each
    // is bounded to its row: a lane whose bytes lie past the row end (K tail, padding segment) or a row >= N reads
    // zeros with no traffic, and an INT4 lane past K also reads scale 0 (its group index is >= G), so no per-lane
    // select is needed.
    int bound_g = -2;
    __amdgpu_buffer_rsrc_t rw[R];
    __amdgpu_buffer_rsrc_t rm[I4 ? R : 1];
    __amdgpu_buffer_rsrc_t rz[F == kI4ZP ? R : 1];
    int nrows = 0;
    auto bind = [&](int g) {
        const int row0 = g < 0 ? 0 : g * R;
        nrows = g < 0 ? 0 : min(R, p.N - row0);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const bool ok = r < nrows;
            const size_t row = (size_t)(row0 + r);
            rw[r] = make_rsrc(p.W + row * row_bytes, ok ? row_bytes : 0u);
            if constexpr (I4) rm[r] = make_rsrc((const uint8_t*)p.meta + row * p.meta_bytes, ok ? p.meta_bytes : 0u);
            if constexpr (F == kI4ZP) rz[r] = make_rsrc(p.zeros + row * p.zbytes, ok ? p.zbytes : 0u);
        }
        bound_g = g;
    };

    // H=0 epilogue operands, loaded once per wave before the streaming loop: lane kk*R + r holds FP8 scale and bias
    // of row r of the wave's group number kk. The launch gives no wave more than ep_groups = 64/R groups, so one
    // load covers them all and the loop holds no conditional load (a load under a branch there makes the compiler
    // wait for every outstanding load, draining the prefetched items at every row). Rows past N read 0.
    constexpr int ep_groups = kWave / R;
    uint32_t ep_scale = 0u, ep_bias = 0u;
    auto ep_load = [&](int k_first) {
        const int kk = lane / R, r = lane - kk * R;
        const int g = it.g0 + (k_first + kk) * it.gstride;
        const bool ok = kk < ep_groups && g < p.ngroups && g * R + r < p.N;
        const uint32_t row = ok ? (uint32_t)(g * R + r) : kOOB >> 2;
        if constexpr (F == kFP8)
            ep_scale = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(p.meta, (uint32_t)p.N * 4u), row * 4u, 0u, 0);
        ep_bias = ld_u16(make_rsrc(p.bias ? p.bias : p.x, p.bias ? (uint32_t)p.N * 2u : 0u), row * 2u, 0u);
    };

    const __amdgpu_buffer_rsrc_t xrs_g = make_rsrc(p.x, XG ? (uint32_t)p.K * 2u : 0u);   // XG: x bounded to K

    // Loads of the item `it` points at into B (size-0 descriptors when there is none: no traffic). Every load is
    // issued unconditionally: a load under a branch would make the compiler wait for every outstanding load,
    // including the other buffer's, before using this item.
    auto issue = [&](Item<F, R, U, XG>& B) {
        const bool ok = it.valid();
        const int g = ok ? it.g : -1;
        if (g != bound_g) bind(g);
        B.group = g;
        B.chunk0 = it.s * U;
        B.k = it.k;
        B.last = !ok || it.s + it.sstep >= it.nseg;
        if constexpr (I4) {
            // the lane's 32 weights of chunk c lie in group c*16 + gl; zero points are packed 2 groups per byte.
            // Issued ahead of the item's weight loads: loads complete in order, so a wait for the scale or zero point
            // never waits for the weights, wherever the compiler places the first use of either (a zero-extension
            // of the zero-point byte at the loop head once made every item wait for its whole load set before any
            // arithmetic).
            const uint32_t moff = gl * 2u + (uint32_t)B.chunk0 * 32u;
            const uint32_t zoff = (gl >> 1) + (uint32_t)B.chunk0 * 8u;
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    B.s[r][u] = ld_u16(rm[r], moff + (uint32_t)u * 32u, 0u);
                    if constexpr (F == kI4ZP) B.z[r][u] = ld_u8(rz[r], zoff + (uint32_t)u * 8u, 0u);
                }
        }
        // one VALU add per buffer; the u-th chunk is an immediate offset of the load
        const uint32_t woff = lane16 + (uint32_t)B.chunk0 * kChunkBytes;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int r = 0; r < R; ++r) B.w[r][u] = ld16<AUX>(rw[r], woff + (uint32_t)u * kChunkBytes, 0u);
        if constexpr (XG) {
            // the lane's x for chunk c: columns c*CC + lane*CPL .. +CPL-1 (CPL = 8*XQ), XQ 16-byte vectors; bounded
            // to K (zeros past it, and for no item at all)
            constexpr uint32_t cpl = 8u * XQ, cc_bytes = 2u * kWave * cpl;
            const uint32_t xoff = ok ? (uint32_t)B.chunk0 * cc_bytes + (uint32_t)lane * (2u * cpl) : kOOB;
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int j = 0; j < XQ; ++j) B.xg[u][j] = ld16<0>(xrs_g, xoff + (uint32_t)u * cc_bytes + 16u * j, 0u);
        }
        it.advance();
    };

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    float accm[R][MB];   // MB > 1: one accumulator per (row, activation row)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MB; ++m) accm[r][m] = 0.0f;
    const int xstride = (int)(xrow / 16u);                   // u32x4 per staged x copy
    const int sstride = (int)(srow / 4u);                    // floats per staged lane-sum copy
    I4Stage st[MB];                                          // INT4 staged x: each activation row's exponent
#pragma unroll
    for (int m = 0; m < MB; ++m) st[m] = {0, 0};

    // Chunks past the row end hold zero weights (and zero INT4 scales); their x index is clamped to the last
    // staged chunk so every product stays 0 * finite.
    auto consume_rows = [&](const Item<F, R, U, XG>& B) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int c = B.chunk0 + u;
            c = c < nchunks ? c : nchunks - 1;
            u32x4 xv[MB][XQ];
#pragma unroll
            for (int m = 0; m < MB; ++m)
#pragma unroll
                for (int j = 0; j < XQ; ++j) xv[m][j] = xs[m * xstride + (c * XQ + j) * kWave + lane];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const u32x4 w = B.w[r][u];
                const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
                if constexpr (F == kBF16) {
#pragma unroll
                    for (int m = 0; m < MB; ++m) accm[r][m] = dot_bf16_16B(w, xv[m][0], accm[r][m]);
                } else if constexpr (F == kFP8) {
                    // decode the 16 weights once (8 bf16 pairs), then one v_dot2 chain per activation row
                    uint32_t d[8];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        d[2 * i] = fp8x2_to_bf16x2<false>(ww[i]);
                        d[2 * i + 1] = fp8x2_to_bf16x2<true>(ww[i]);
                    }
#pragma unroll
                    for (int m = 0; m < MB; ++m) {
                        const uint32_t xa[8] = {xv[m][0].x, xv[m][0].y, xv[m][0].z, xv[m][0].w,
                                                xv[m][1].x, xv[m][1].y, xv[m][1].z, xv[m][1].w};
                        float a = accm[r][m];
#pragma unroll
                        for (int i = 0; i < 8; ++i) a = dot2_bf16(d[i], xa[i], a);
                        accm[r][m] = a;
                    }
                } else {
                    float dm[MB];
#pragma unroll
                    for (int m = 0; m < MB; ++m) dm[m] = 0.0f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {   // word i: 8 nibbles -> 4 bf16 subnormal pairs, then MB dot chains
                        uint32_t q4[4];
                        i4_word_decode_dn(ww[i], q4);
#pragma unroll
                        for (int m = 0; m < MB; ++m) {
                            const u32x4 xw = xv[m][i];
                            dm[m] = dot2_bf16(q4[0], xw.x, dm[m]);
                            dm[m] = dot2_bf16(q4[1], xw.y, dm[m]);
                            dm[m] = dot2_bf16(q4[2], xw.z, dm[m]);
                            dm[m] = dot2_bf16(q4[3], xw.w, dm[m]);
                        }
                    }
                    float s, zc;
                    if constexpr (F == kI4) {
                        s = f16_to_f32(B.s[r][u]);
                        zc = 8.0f;                                // the format's zero point
                    } else {
                        s = bf16_to_f32(B.s[r][u]);
                        zc = (float)((B.z[r][u] >> (gl & 1u) * 4u) & 0xFu);
                    }
#pragma unroll
                    for (int m = 0; m < MB; ++m) {
                        const float sx = s32[m * sstride + c * kWave + lane];
                        accm[r][m] = __builtin_fmaf(s, __builtin_fmaf(-zc, sx, dm[m]), accm[r][m]);
                    }
                }
            }
        }
    };

    auto consume = [&](const Item<F, R, U, XG>& B) {
        if constexpr (MB > 1) {
            consume_rows(B);
            return;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int c = B.chunk0 + u;
            c = c < nchunks ? c : nchunks - 1;
            u32x4 xv[XQ];
            float sx_g = 0.0f;   // XG, INT4: the lane's 32-column x sum, in the staged order (s0 + s1) + (s2 + s3)
            if constexpr (XG) {
                float s8[XQ];
#pragma unroll
                for (int j = 0; j < XQ; ++j) {
                    xv[j] = B.xg[u][j];
                    if constexpr (I4) s8[j] = i4_pair_sum_x(xv[j]);
                }
                if constexpr (I4) sx_g = (s8[0] + s8[1]) + (s8[2] + s8[3]);
            } else {
#pragma unroll
                for (int j = 0; j < XQ; ++j) xv[j] = xs[(c * XQ + j) * kWave + lane];
            }
            if constexpr (F == kBF16) {
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] = dot_bf16_16B(B.w[r][u], xv[0], acc[r]);
            } else if constexpr (F == kFP8) {
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] = dot_fp8_16B(B.w[r][u], xv[0], xv[1], acc[r]);
            } else {
                // staged x: the subnormal decode, dot and x sum in units of 2^unit, no decode offset; XG and D43:
                // the 0x43-exponent decode against unscaled x, offset 128
                const float sx = XG ? sx_g : s32[c * kWave + lane];
                constexpr float off = DN ? 0.0f : 128.0f;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float d = DN ? dot_i4dn_16B(B.w[r][u], xv[0], xv[1], xv[2], xv[3])
                                       : dot_i4_16B(B.w[r][u], xv[0], xv[1], xv[2], xv[3], c43);
                    float s, zc;
                    if constexpr (F == kI4) {
                        s = f16_to_f32(B.s[r][u]);
                        zc = off + 8.0f;                          // decode offset + the format's zero point
                    } else {
                        s = bf16_to_f32(B.s[r][u]);
                        const uint32_t z = (B.z[r][u] >> (gl & 1u) * 4u) & 0xFu;
                        zc = off + (float)z;
                    }
                    acc[r] = __builtin_fmaf(s, __builtin_fmaf(-zc, sx, d), acc[r]);
                }
            }
        }
    };

    // End of a group for this wave: reduce over the wave, then store (H=0) or park the partial in LDS (H=1).
    // MB > 1: reduce the R x MB sums (two per paired wave reduction), then lanes kk*R + r store row r's MB outputs
    auto finish_rows = [&](const Item<F, R, U, XG>& B) {
        constexpr int NV = R * MB;
        float flat[NV], tot[NV];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                flat[r * MB + m] = accm[r][m];
                accm[r][m] = 0.0f;
            }
#pragma unroll
        for (int i = 0; i + 1 < NV; i += 2) {
            const float v = wave_sum2(flat[i], flat[i + 1]);
            tot[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
            tot[i + 1] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
        }
        if constexpr (NV & 1) tot[NV - 1] = wave_sum(flat[NV - 1]);
        if constexpr (DN) {   // back from the subnormal decode's units of 2^unit (exact: a power of two)
#pragma unroll
            for (int i = 0; i < NV; ++i) tot[i] = ldexp_f32(tot[i], -st[i % MB].unit);
        }
        const int kk = B.k;
        const int r = lane - kk * R;
        const int row = B.group * R + r;
        if (r >= 0 && r < R && row < p.N) {
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                float v = tot[m];
#pragma unroll
                for (int i = 1; i < R; ++i) v = r == i ? tot[i * MB + m] : v;
                if constexpr (F == kFP8) v = v * __uint_as_float(ep_scale);
                if (p.bias) v = v + bf16_to_f32(ep_bias);
                p.y[(size_t)m * (size_t)p.N + row] = (uint16_t)f32_to_bf16_out(v);
            }
        }
    };

    auto finish = [&](const Item<F, R, U, XG>& B) {
        if constexpr (MB > 1) {
            finish_rows(B);
            return;
        }
        float tot[R];
#pragma unroll
        for (int r = 0; r + 1 < R; r += 2) {
            const float v = wave_sum2(acc[r], acc[r + 1]);
            tot[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
            tot[r + 1] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
        }
        if constexpr (R & 1) tot[R - 1] = wave_sum(acc[R - 1]);
        if constexpr (DN) {   // back from the subnormal decode's units of 2^unit (exact: a power of two)
#pragma unroll
            for (int r = 0; r < R; ++r) tot[r] = ldexp_f32(tot[r], -st[0].unit);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
        if constexpr (!KSPLIT) {
            // lanes kk*R .. kk*R+R-1 hold this group's epilogue operands (kk = the group's slot in the window) and
            // store its R rows: one store instruction per group
            const int kk = B.k;   // < ep_groups (launch_gemv caps the groups per wave)
            const int r = lane - kk * R;
            float v = tot[0];
#pragma unroll
            for (int i = 1; i < R; ++i) v = r == i ? tot[i] : v;
            const int row = B.group * R + r;
            if (r >= 0 && r < R && row < p.N) {
                if constexpr (F == kFP8) v = v * __uint_as_float(ep_scale);
                if (p.bias) v = v + bf16_to_f32(ep_bias);
                p.y[row] = (uint16_t)f32_to_bf16_out(v);
            }
        } else {
            if (lane < R) {
                float v = tot[0];
#pragma unroll
                for (int r = 1; r < R; ++r) v = lane == r ? tot[r] : v;
                part[((B.k % p.round) * W + wave) * R + lane] = v;
            }
        }
    };

    // H=1: combine the parked partials of the groups of the round that ends with group index k_end (exclusive),
    // in wave order, and store.
    auto combine = [&](int k_begin, int k_end) {
        __syncthreads();
        const int n = (k_end - k_begin) * R;
        const int wn = min(W, p.nseg);   // waves that own a segment (and so parked a partial) in every group
        for (int i = (int)threadIdx.x; i < n; i += W * kWave) {
            const int kk = i / R, r = i - kk * R;
            const int row = ((int)blockIdx.x + (k_begin + kk) * (int)gridDim.x) * R + r;
            const int slot = (k_begin + kk) % p.round;
            float v = 0.0f;
            for (int w = 0; w < wn; ++w) v += part[(slot * W + w) * R + r];
            if (row < p.N) {
                if constexpr (F == kFP8) v = v * reinterpret_cast<const float*>(p.meta)[row];
                if (p.bias) v = v + bf16_to_f32(p.bias[row]);
                p.y[row] = (uint16_t)f32_to_bf16_out(v);
            }
        }
        __syncthreads();
    };

    // x loads first (ahead of the weight loads in the memory queues), then all D item buffers, then x into LDS.
    // All D buffers are in flight while x is staged, so a small GEMV (a few items per wave) costs one memory round
    // trip. From then on, the buffer just consumed is refilled with the item D places further on (D = 2).
    // early x vectors per thread: 16 KiB of x per block, 32 KiB for the one-block-per-CU W = 16 launch (no other
    // block's weight loads can queue ahead of its x, and K up to 16384 is then staged without late loads)
    // (MB > 1: the same early budget shared over the MB activation rows, at least one vector per thread each)
    constexpr int XE0 = (W >= 16 ? 2048 : 1024) / (W * kWave);
    constexpr int XE = MB == 1 ? XE0 : (XE0 / MB > 0 ? XE0 / MB : 1);
    constexpr int D = pipe_depth<R, U>();
    XRegs<XE> xr[MB];
    if constexpr (!XG) {
#pragma unroll
        for (int m = 0; m < MB; ++m) x_load<F, XE, W * kWave>(p.x + (size_t)m * (size_t)p.K, p.K, xr[m]);
    }
    if constexpr (!KSPLIT) ep_load(0);
    Item<F, R, U, XG> buf[D];
#pragma unroll
    for (int d = 0; d < D; ++d) issue(buf[d]);
    if constexpr (!XG) {
        // INT4, subnormal decode: x is staged at the first scale (kI4StageFirst) with integer operations, and each
        // wave parks its window flags per activation row in LDS; after the barrier every wave reads the block's (the
        // row's: every block stages the whole row). A row whose x lies outside the first scale's window is staged
        // again at the scale its largest |x| calls for (i4_stage_exp), behind two more barriers. The decision is the
        // same in every wave and block. The 0x43 decode (D43) stages x unscaled and needs no window.
        uint32_t tmax[MB];
#pragma unroll
        for (int m = 0; m < MB; ++m) {
            tmax[m] = x_store<F, XE, W * kWave, D43 ? kStage43 : kStageFirst>(
                p.x + (size_t)m * (size_t)p.K, p.K, nchunks, xr[m], xs + m * xstride, s32 + m * sstride);
            if constexpr (DN) {
                const uint32_t f = i4_window_flags(tmax[m]);
                if (lane == 0) flags[m * 16 + wave] = (uint8_t)f;
                st[m] = kI4StageFirst;
            }
        }
        __syncthreads();
        if constexpr (DN) {
            bool again = false, redo[MB];
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                const uint32_t f = (uint32_t)__builtin_amdgcn_readfirstlane((int)or_flag_bytes<W>(flags + m * 16));
                redo[m] = !i4_first_stands(f);
                again = again || redo[m];
            }
            if (again) {
#pragma unroll
                for (int m = 0; m < MB; ++m) {
                    const uint32_t mw = wave_max_u32(tmax[m]);
                    if (redo[m] && lane == 0) maxima[m * W + wave] = mw;
                }
                __syncthreads();
#pragma unroll
                for (int m = 0; m < MB; ++m) {
                    if (!redo[m]) continue;
                    uint32_t mx = 0u;
#pragma unroll
                    for (int w = 0; w < W; ++w) mx = max(mx, maxima[m * W + w]);
                    st[m] = i4_stage_exp((uint32_t)__builtin_amdgcn_readfirstlane((int)mx));
                    x_restage<F, W * kWave>(p.x + (size_t)m * (size_t)p.K, p.K, nchunks, xs + m * xstride,
                                            s32 + m * sstride, st[m].a);
                }
                __syncthreads();
            }
        }
    }

    // The loops leave by `return` when the wave's items run out (nothing follows them): an exit that rejoined the
    // loop header without the other buffer's loads would make the compiler's wait counts assume those loads absent,
    // and every consume would then wait for all outstanding loads (vmcnt(0)), the prefetched item included.
    // The drain kernels (DR: launches whose waves take at most two items) leave the walk for a drain instead, once it
    // has no item left to issue: issuing the empty item's loads (size-0 descriptors, no traffic) kept the wave
    // waiting behind every outstanding request of its CU (per-wave timestamps: a median 0.68 us between the last
    // item and the exit on FP8 4096x4096, 0.12 us with the drain on INT4 4096x4096). The drain loop's second exit
    // costs a register copy and a vmcnt(0) on its back edge, which never runs at two items per wave but was slower
    // with more (FP8 28672x4096 +0.67 us, INT4 37888x3584 +0.85 us, INT4 4096x14336 +0.11): those keep the plain loop.
    if constexpr (!KSPLIT && DR) {
        auto step = [&](const Item<F, R, U, XG>& B) {
            consume(B);
            if (B.last) finish(B);
        };
        static_assert(D == 2, "the drains below follow two buffers");
        for (;;) {
            if (buf[0].group < 0) return;   // a wave without items
            step(buf[0]);
            if (!it.valid()) goto drain0;
            issue(buf[0]);
            if (buf[1].group < 0) return;   // a wave with one item
            step(buf[1]);
            if (!it.valid()) goto drain1;
            issue(buf[1]);
        }
    drain0:   // buf[0] was the walk's last but one item or none: buf[1] holds the last, if any
        if (buf[1].group >= 0) step(buf[1]);
        return;
    drain1:
        if (buf[0].group >= 0) step(buf[0]);
        return;
    } else if constexpr (!KSPLIT) {
        for (;;) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                if (buf[d].group < 0) return;
                consume(buf[d]);
                if (buf[d].last) finish(buf[d]);
                issue(buf[d]);
            }
        }
    } else {
        // The block's groups, in rounds of p.round; every wave walks the same groups (with its own segments), so
        // the per-round barriers are reached by all waves. Waves without a segment (wave >= nseg) only combine.
        const int ngb = (int)blockIdx.x < p.ngroups ? (p.ngroups - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
        int k_done = 0;
        if (buf[0].group >= 0) {
            for (;;) {
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    if (buf[d].group < 0) return;   // every round this wave takes part in is combined by now
                    consume(buf[d]);
                    if (buf[d].last) {
                        finish(buf[d]);
                        const int k_cur = buf[d].k + 1;   // groups parked so far
                        if (k_cur - k_done == p.round || k_cur == ngb) {
                            combine(k_done, k_cur);
                            k_done = k_cur;
                        }
                    }
                    issue(buf[d]);
                }
            }
        } else {
            // no segment for this wave: still take part in every round's barriers
            for (int k0 = 0; k0 < ngb; k0 += p.round) {
                const int k1 = min(ngb, k0 + p.round);
                combine(k0, k1);
            }
        }
    }
}

template <int F, int R, int U, int W, int AUX, bool KSPLIT>
__global__ void __launch_bounds__(W * kWave) gemv_kernel(GemvParams p)
{
    gemv_body<F, R, U, W, AUX, KSPLIT, 1>(p);
}

// The same, ending in a drain (H = 0 launches whose waves take at most two items).
template <int F, int R, int U, int W, int AUX, bool KSPLIT>
__global__ void __launch_bounds__(W * kWave) gemv_kernel_dr(GemvParams p)
{
    gemv_body<F, R, U, W, AUX, KSPLIT, 1, false, false, true>(p);
}

// INT4, M = 1, staged x for the 0x43-exponent decode (the launch's waves make few weight loads).
template <int F, int R, int U, int W, int AUX, bool KSPLIT>
__global__ void __launch_bounds__(W * kWave) gemv_kernel43(GemvParams p)
{
    gemv_body<F, R, U, W, AUX, KSPLIT, 1, false, true>(p);
}

// The same, ending in a drain.
template <int F, int R, int U, int W, int AUX, bool KSPLIT>
__global__ void __launch_bounds__(W * kWave) gemv_kernel43_dr(GemvParams p)
{
    gemv_body<F, R, U, W, AUX, KSPLIT, 1, false, true, true>(p);
}

// x from global memory (K beyond what the LDS can stage), M = 1.
template <int F, int R, int U, int W, int AUX, bool KSPLIT>
__global__ void __launch_bounds__(W * kWave) gemv_kernel_xg(GemvParams p)
{
    gemv_body<F, R, U, W, AUX, KSPLIT, 1, true>(p);
}

// Small batch on the M = 1 design: MB = 2..6 (BF16 and FP8 2..8) activation rows, row-parallel (no split-K).
template <int F, int R, int U, int W, int AUX, int MB>
__global__ void __launch_bounds__(W * kWave) gemv_rows_kernel(GemvParams p)
{
    gemv_body<F, R, U, W, AUX, false, MB>(p);
}

// ---------------------------------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------------------------------

// Device facts used to size the persistent grid (queried once; the library assumes one GPU model per process).
struct DeviceFacts {
    int cus = 0;
    int lds_per_cu = 0;
    int lds_per_block = 0;
};
DeviceFacts device_facts();

// Resident waves per CU the persistent grid aims for (each block stages x, so more blocks mean more x traffic). A
// 16-wave block runs alone on its CU: staging x once per CU, ahead of every weight load there, is what it is for.
#ifndef PAIA_GEMV_MAX_WAVES_PER_CU
#define PAIA_GEMV_MAX_WAVES_PER_CU 32
#endif
constexpr int kMaxWavesPerCu = PAIA_GEMV_MAX_WAVES_PER_CU;
template <int W>
constexpr int max_blocks_per_cu_for()
{
    return W >= 16 ? 1 : (kMaxWavesPerCu / W > 0 ? kMaxWavesPerCu / W : 1);
}

// Largest LDS a launch may request (bytes). Beyond it the entry points return -2.
constexpr uint32_t kMaxLds = 65536;
// LDS for split-K partials (H=1): up to this much, within kMaxLds; at least one group (W*R floats) is needed.
constexpr uint32_t kPartBytes = 8192;

// LDS of an M = 1 launch of format F with R rows per group, W waves per block, split-K or not, and (split-K) the
// number of row groups per combine round. Returns 0 when x does not fit (the launch then loads x from global memory).
// The one plan both the launch and paia_gemv_pick_variant (which prefers variants that stage x) go by.
inline uint32_t lds_plan(int F, int R, int W, bool ksplit, int nchunks, int* round)
{
    *round = 1;
    const bool i4 = F == kI4 || F == kI4ZP;
    const uint64_t xq = F == kBF16 ? 1u : F == kFP8 ? 2u : 4u;
    // x plus INT4 sums: (XQ*1024 + 256) bytes per chunk; 64-bit (nchunks reaches 2^22 at K = 2^31)
    const uint64_t base64 = (uint64_t)nchunks * (xq * kChunkBytes + (i4 ? kWave * 4u : 0u)) + lds_slot_bytes(F, 1, W);
    if (base64 > kMaxLds) return 0;
    const uint32_t base = (uint32_t)base64;
    if (!ksplit) return base;
    const uint32_t group_bytes = (uint32_t)(W * R * 4);
    uint32_t part = kMaxLds - base < kPartBytes ? kMaxLds - base : kPartBytes;
    part -= part % group_bytes;
    if (part < group_bytes) return 0;
    *round = (int)(part / group_bytes);
    return base + part;
}
template <int F, int R, int W, bool KSPLIT>
uint32_t gemv_lds_plan(int nchunks, int* round)
{
    return lds_plan(F, R, W, KSPLIT, nchunks, round);
}

// Resident blocks per CU the occupancy calculator allows for a kernel (queried once per kernel).
template <typename KernelT>
int max_blocks_per_cu_of(KernelT kernel, int threads, std::atomic<int>& cached)
{
    int v = cached.load(std::memory_order_relaxed);
    if (v == 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess || n <= 0) n = 1;
        cached.store(n, std::memory_order_relaxed);
        v = n;
    }
    return v;
}

template <int F, int R, int U, int W, int AUX, bool KSPLIT>
int gemv_max_blocks_per_cu()
{
    static std::atomic<int> cached{0};
    return max_blocks_per_cu_of(gemv_kernel<F, R, U, W, AUX, KSPLIT>, W * kWave, cached);
}

// The busiest CU's row groups when `grid` blocks of W waves take `ng` groups in rounds of grid*W (block b, wave w
// takes groups b*W + w + k*grid*W), block b running on CU b mod cus. That is CU 0: it holds the most blocks, and its
// j-th block (b = j*cus) has the lowest index of all j-th blocks, so the last round reaches it first.
inline int busiest_cu_groups(int ng, int grid, int W, int cus)
{
    const int full = ng / (grid * W), rem = ng - full * grid * W;
    int load = 0;
    for (int b = 0; b < grid; b += cus) {
        const int tail = rem - b * W;
        load += W * full + (tail <= 0 ? 0 : (tail < W ? tail : W));
    }
    return load;
}

// Persistent grid of a launch: blocks resident at once (occupancy, LDS, the waves-per-CU cap), then the groups per
// wave (H=0) or per block (H=1) that cover N, at most 64/R per wave for H=0 so a wave's epilogue operands fit one
// register (beyond that the grid grows past one resident wave of blocks). H=0 with several blocks per CU and several
// rounds: a whole number of blocks on every CU when that lowers the busiest CU's groups (the fewest blocks covering N
// in q rounds leave some CUs a block more than others: BF16 gate_up 28672x4096 at 3.5 blocks per CU took 38.5 µs,
// at 4 blocks per CU 35.2).
// Split-K launches whose rows are one segment long (U KiB covers a whole row: the lm_heads at U = 8 in BF16) leave
// every wave but the first of a block without a segment, so one wave per block streams whole row groups. For BF16
// (a bare v_dot2 per 4 bytes of weights) 2 such blocks per CU stream fastest: on MI355X, BF16 lm_head 152064x3584 at
// R=1 U=8 W=4 takes 153.1 µs at 2 blocks per CU, 158.6 at 4; 128256x4096 at R=2 U=8 W=8 144.1 and 144.6 (a read
// probe of the walk: 143-147 µs per 1.05-1.09 GB at 2, 144-149 at 4). The FP8 and INT4 decodes cost more per byte
// and want more one-wave blocks per CU (FP8 128256x4096 at R=1 U=4 W=4: 74.9 µs at 4, 129.7 at 2), so they keep the
// general sizing.
#ifndef PAIA_GEMV_LEAD_WAVE_BLOCKS_PER_CU
#define PAIA_GEMV_LEAD_WAVE_BLOCKS_PER_CU 2
#endif
constexpr int kLeadWaveBlocksPerCu = PAIA_GEMV_LEAD_WAVE_BLOCKS_PER_CU;

// lead_cap: blocks per CU for a one-segment split-K launch (0: no cap).
template <int R, int W, bool KSPLIT>
int gemv_grid(const GemvParams& p, uint32_t lds, int per_cu, int lead_cap = 0)
{
    const DeviceFacts df = device_facts();
    if (df.lds_per_cu > 0) {
        const int by_lds = (int)(df.lds_per_cu / (lds ? lds : 1u));
        if (by_lds < per_cu) per_cu = by_lds > 0 ? by_lds : 1;
    }
    if (per_cu > max_blocks_per_cu_for<W>()) per_cu = max_blocks_per_cu_for<W>();
    if (KSPLIT && p.nseg == 1 && lead_cap > 0 && per_cu > lead_cap) per_cu = lead_cap;
    const int cus = df.cus > 0 ? df.cus : 256;
    const int gmax = cus * per_cu;
    const int ng = p.ngroups;
    // units of work dealt round-robin: row groups to waves (H=0) or to blocks (H=1)
    const int per_block_units = KSPLIT ? 1 : W;
    int grid = (ng + per_block_units - 1) / per_block_units;
    if (grid > gmax) grid = gmax;
    int q = (ng + grid * per_block_units - 1) / (grid * per_block_units);   // units per wave / block
    if (!KSPLIT && q > kWave / R) q = kWave / R;
    const int fewest = (ng + q * per_block_units - 1) / (q * per_block_units);
    if (KSPLIT || per_cu < 2 || q < 2) return fewest;
    int b = ((ng + cus - 1) / cus + q * W - 1) / (q * W);   // blocks per CU for its share in q rounds
    if (b > per_cu) b = per_cu;
    const int even = cus * b;
    if ((ng + even * W - 1) / (even * W) > q) return fewest;
    return busiest_cu_groups(ng, even, W, cus) < busiest_cu_groups(ng, fewest, W, cus) ? even : fewest;
}

// The launch for K whose staged x does not fit the LDS: x comes from global memory with each item's weights
// (gemv_kernel_xg), split-K over the 8 waves of a block, one row per group, 2 KiB of each row per item; the LDS holds
// only the split-K partials. Every variant of a format runs this kernel at such K (the knobs of the call are not
// used), so any K the format's alignment rules accept runs. Returns 0 or a hipError_t.
template <int F, int R, int U, int W, int AUX, bool KSPLIT>
int launch_gemv_xg_knobs(GemvParams p, hipStream_t st)
{
    p.nchunks = (int)((p.row_bytes + kChunkBytes - 1) / kChunkBytes);
    p.nseg = (p.nchunks + U - 1) / U;
    p.ngroups = (p.N + R - 1) / R;
    p.round = KSPLIT ? (int)(kPartBytes / (uint32_t)(W * R * 4)) : 1;
    const uint32_t lds = KSPLIT ? kPartBytes : 0u;
    static std::atomic<int> cached{0};
    const int per_cu = max_blocks_per_cu_of(gemv_kernel_xg<F, R, U, W, AUX, KSPLIT>, W * kWave, cached);
    const int grid = gemv_grid<R, W, KSPLIT>(p, lds, per_cu);
    hipLaunchKernelGGL((gemv_kernel_xg<F, R, U, W, AUX, KSPLIT>), dim3(grid), dim3(W * kWave), lds, st, p);
    return (int)hipGetLastError();
}

template <int F, int AUX>
int launch_gemv_xg(GemvParams p, hipStream_t st)
{
    return launch_gemv_xg_knobs<F, 1, 2, 8, AUX, true>(p, st);
}

// INT4 with staged x: launches whose waves make at most this many 16-byte weight loads run the 0x43-exponent decode
// against unscaled x (gemv_kernel43); the others the subnormal decode. The subnormal decode takes 5 VALU per 8 weights
// against the 0x43 decode's 7, but its staging scales x and checks the row's range before any item is consumed, a
// prologue that precedes the first item on every wave; with few items per wave the prologue weighs more. Measured on
// MI355X (per launch, 0x43 / subnormal decode, loads per wave in brackets): asymmetric format Llama qkv 6144x4096 (2)
// 4.74 / 4.93 us, o 4096x4096 (2) 3.96 / 4.09, down 4096x14336 (7) 7.16 / 7.28, gate_up 28672x4096 (8) 12.11 / 12.18,
// Qwen qkv 4608x3584 (2) 4.55 / 4.75, down 3584x18944 (10) 8.94 / 8.61, gate_up 37888x3584 (20) 14.02 / 13.35;
// reference format down (7) 7.09 / 7.21, gate_up (8) 11.85 / 11.50.
constexpr int kI4Max43Loads = 7;

// 16-byte weight loads per wave (per lane) of a launch of `grid` blocks: the groups a wave (H=0) or block (H=1) takes,
// times the segments a wave takes of each, times R * U loads per item.
inline int loads_per_wave(const GemvParams& p, int grid, int R, int U, int W, bool ksplit)
{
    if (grid <= 0) return 0;
    if (!ksplit) return ((p.ngroups + grid * W - 1) / (grid * W)) * p.nseg * R * U;
    return ((p.ngroups + grid - 1) / grid) * ((p.nseg + W - 1) / W) * R * U;
}

template <int F, int R, int U, int W, int AUX, bool KSPLIT>
int gemv43_max_blocks_per_cu()
{
    static std::atomic<int> cached{0};
    return max_blocks_per_cu_of(gemv_kernel43<F, R, U, W, AUX, KSPLIT>, W * kWave, cached);
}

// Whether the drain kernel of a launch planned for its plain twin holds the same grid resident at once (the drain
// kernels use more registers; a grid that no longer fits in one round would queue blocks behind the first round).
template <int F, int R, int U, int W, int AUX, bool KSPLIT, bool K43>
bool drain_fits(int grid)
{
    if constexpr (KSPLIT) {
        return false;
    } else {
        static std::atomic<int> cached{0};
        int per_cu = 0;
        if constexpr (K43) per_cu = max_blocks_per_cu_of(gemv_kernel43_dr<F, R, U, W, AUX, KSPLIT>, W * kWave, cached);
        else per_cu = max_blocks_per_cu_of(gemv_kernel_dr<F, R, U, W, AUX, KSPLIT>, W * kWave, cached);
        const DeviceFacts df = device_facts();
        return grid <= (df.cus > 0 ? df.cus : 256) * per_cu;
    }
}

// The kernel a launch runs: 0 gemv_kernel, 1 gemv_kernel43 (INT4, few loads per wave), 2 gemv_kernel_xg (x beyond the
// LDS), 3 gemv_kernel_dr and 4 gemv_kernel43_dr (the same two ending in a drain: H = 0, at most two items per wave).
// p as the entry point fills it; sets p's derived fields and *lds, *grid for the chosen kernel.
template <int F, int R, int U, int W, int AUX, bool KSPLIT>
int gemv_plan(GemvParams& p, uint32_t* lds, int* grid)
{
    p.nchunks = (int)((p.row_bytes + kChunkBytes - 1) / kChunkBytes);
    p.nseg = (p.nchunks + U - 1) / U;
    p.ngroups = (p.N + R - 1) / R;
    *lds = gemv_lds_plan<F, R, W, KSPLIT>(p.nchunks, &p.round);
    if (*lds == 0) return 2;
    if constexpr ((F == kI4 || F == kI4ZP) && R * U <= 2) {
        const int g43 = gemv_grid<R, W, KSPLIT>(p, *lds, gemv43_max_blocks_per_cu<F, R, U, W, AUX, KSPLIT>());
        const int n = loads_per_wave(p, g43, R, U, W, KSPLIT);
        if (n <= kI4Max43Loads) {
            *grid = g43;
            return !KSPLIT && n <= 2 * R * U && drain_fits<F, R, U, W, AUX, KSPLIT, true>(g43) ? 4 : 1;
        }
    }
    *grid = gemv_grid<R, W, KSPLIT>(p, *lds, gemv_max_blocks_per_cu<F, R, U, W, AUX, KSPLIT>(),
                                    F == kBF16 ? kLeadWaveBlocksPerCu : 0);
    const bool two = loads_per_wave(p, *grid, R, U, W, KSPLIT) <= 2 * R * U;   // at most two items per wave
    return !KSPLIT && two && drain_fits<F, R, U, W, AUX, KSPLIT, false>(*grid) ? 3 : 0;
}

// Launch on `st`. Arguments were validated by the caller. Returns 0 or a hipError_t. K whose staged x (and, H=1, one
// round of partials) does not fit the LDS runs launch_gemv_xg instead.
template <int F, int R, int U, int W, int AUX, bool KSPLIT>
int launch_gemv(GemvParams p, hipStream_t st)
{
    uint32_t lds = 0;
    int grid = 0;
    const int k = gemv_plan<F, R, U, W, AUX, KSPLIT>(p, &lds, &grid);
    if (k == 2) return launch_gemv_xg<F, AUX>(p, st);
    if constexpr ((F == kI4 || F == kI4ZP) && R * U <= 2) {
        if (k == 1) {
            hipLaunchKernelGGL((gemv_kernel43<F, R, U, W, AUX, KSPLIT>), dim3(grid), dim3(W * kWave), lds, st, p);
            return (int)hipGetLastError();
        }
        if constexpr (!KSPLIT) {
            if (k == 4) {
                hipLaunchKernelGGL((gemv_kernel43_dr<F, R, U, W, AUX, KSPLIT>), dim3(grid), dim3(W * kWave), lds, st,
                                   p);
                return (int)hipGetLastError();
            }
        }
    }
    if constexpr (!KSPLIT) {
        if (k == 3) {
            hipLaunchKernelGGL((gemv_kernel_dr<F, R, U, W, AUX, KSPLIT>), dim3(grid), dim3(W * kWave), lds, st, p);
            return (int)hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemv_kernel<F, R, U, W, AUX, KSPLIT>), dim3(grid), dim3(W * kWave), lds, st, p);
    return (int)hipGetLastError();
}

// Which kernel a launch of this variant runs (gemv_plan's first result), for tools that name it.
template <int F, int R, int U, int W, int AUX, bool KSPLIT>
int gemv_kernel_kind(GemvParams p)
{
    uint32_t lds = 0;
    int grid = 0;
    return gemv_plan<F, R, U, W, AUX, KSPLIT>(p, &lds, &grid);
}

// LDS the row-streaming launch may request: the device's per-block limit (160 KiB on MI355X), at least kMaxLds. A block
// that large runs alone on its CU, which suits the 16-wave variants.
inline uint32_t rows_max_lds()
{
    const int l = device_facts().lds_per_block;
    return l > (int)kMaxLds ? (uint32_t)l : kMaxLds;
}

// The row-streaming small-batch launch: MB activation rows (x [MB][K], y [MB][N]); LDS holds MB copies of the
// staged x (and INT4 lane sums). Returns -2 when they exceed rows_max_lds().
template <int F, int R, int U, int W, int AUX, int MB>
int launch_gemv_rows(GemvParams p, hipStream_t st)
{
    p.nchunks = (int)((p.row_bytes + kChunkBytes - 1) / kChunkBytes);
    p.nseg = (p.nchunks + U - 1) / U;
    p.ngroups = (p.N + R - 1) / R;
    p.round = 1;
    const uint64_t lds = (uint64_t)MB * (lds_x_bytes<F>(p.nchunks) + lds_s32_bytes<F>(p.nchunks)) +
                         lds_slot_bytes(F, MB, W);
    if (lds > rows_max_lds()) return -2;
    if (lds > kMaxLds) {   // beyond the default dynamic-LDS limit: raise it once for this kernel
        static std::atomic<int> raised{0};
        if (!raised.load(std::memory_order_relaxed)) {
            const hipError_t e = hipFuncSetAttribute(
                reinterpret_cast<const void*>(&gemv_rows_kernel<F, R, U, W, AUX, MB>),
                hipFuncAttributeMaxDynamicSharedMemorySize, (int)rows_max_lds());
            if (e != hipSuccess) return (int)e;
            raised.store(1, std::memory_order_relaxed);
        }
    }
    static std::atomic<int> cached{0};
    const int per_cu = max_blocks_per_cu_of(gemv_rows_kernel<F, R, U, W, AUX, MB>, W * kWave, cached);
    const int grid = gemv_grid<R, W, false>(p, (uint32_t)lds, per_cu);
    hipLaunchKernelGGL((gemv_rows_kernel<F, R, U, W, AUX, MB>), dim3(grid), dim3(W * kWave), (uint32_t)lds, st, p);
    return (int)hipGetLastError();
}

using GemvLaunchFn = int (*)(GemvParams, hipStream_t);
using GemvKindFn = int (*)(GemvParams);

// The M = 1 kernel of a format with the library's variant for (N, K) (paia_gemv_pick_variant), p filled as that
// format's M = 1 entry point fills it; 0, -2 (LDS limit) or a hipError_t. The small-batch entry points use these at
// M = 1. zp: the asymmetric INT4 format.
int launch_gemv_bf16_picked(GemvParams p, hipStream_t st);
int launch_gemv_fp8_picked(GemvParams p, hipStream_t st);
int launch_gemv_int4_picked(GemvParams p, bool zp, hipStream_t st);

struct Variant {
    int R, U, W, S, H;
    GemvLaunchFn fn;
    GemvKindFn kind;   // which kernel a launch runs (gemv_kernel_kind)
};

// The kernel a launch of table variant v would run for p (N, K, row_bytes and the format's sizes filled): 0
// gemv_kernel, 1 gemv_kernel43, 2 gemv_kernel_xg; -1 for a variant outside the table. zp: the asymmetric INT4 format.
int kind_bf16(int v, GemvParams p);
int kind_fp8(int v, GemvParams p);
int kind_int4(int v, bool zp, GemvParams p);

inline bool aligned(const void* ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0; }

}  // namespace paia
