// Device helpers for the gfx950 (CDNA4) GEMV kernels: buffer-resource loads, format decode + dot products on the
// VALU, wave64 reductions, and the bf16 round-to-nearest-even used by every epilogue.
//
// Everything here is written for wave64 gfx950 only. Weight rows are read with raw buffer loads whose descriptor is
// bounded to the row, so loads past the end of a row (K tails, rows >= N) return zeros without a branch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace paia {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------------------------------
// weight formats
// ---------------------------------------------------------------------------------------------------------------
enum Fmt : int {
    kBF16 = 0,   // W bf16 [N][K]
    kFP8 = 1,    // W e4m3fn [N][K], fp32 scale per row
    kI4 = 2,     // W uint4 [N][K/2] (z = 8), fp16 scale [N][K/128]         (reference format)
    kI4ZP = 3,   // W uint4 [N][K/2], bf16 scale [N][G], 4-bit zero [N][ceil(G/2)] (asymmetric format)
};

// Per format: weight columns covered by one 16-byte load, and how many 16-byte LDS x vectors (8 bf16 each) they need.
template <int F> struct FmtInfo;
template <> struct FmtInfo<kBF16> { static constexpr int kColsPer16B = 8;  static constexpr int kXQ = 1; };
template <> struct FmtInfo<kFP8>  { static constexpr int kColsPer16B = 16; static constexpr int kXQ = 2; };
template <> struct FmtInfo<kI4>   { static constexpr int kColsPer16B = 32; static constexpr int kXQ = 4; };
template <> struct FmtInfo<kI4ZP> { static constexpr int kColsPer16B = 32; static constexpr int kXQ = 4; };

// A "chunk" is what one wave reads from one weight row with one 16-byte load per lane: 1 KiB.
constexpr int kWave = 64;
constexpr int kChunkBytes = kWave * 16;

// ---------------------------------------------------------------------------------------------------------------
// buffer resources (gfx9 family: dword3 = 0x00020000, raw buffer, no swizzle)
// ---------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t nbytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes, 0x00020000);
}

// aux = cache policy: 0 default, 2 = nt (streaming; the weights are read exactly once per call).
template <int AUX>
__device__ __forceinline__ u32x4 ld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, AUX));
}
__device__ __forceinline__ uint32_t ld_u16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}
__device__ __forceinline__ uint32_t ld_u8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, voff, soff, 0);
}

// ---------------------------------------------------------------------------------------------------------------
// arithmetic
// ---------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc)
{
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), acc, false);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }

__device__ __forceinline__ float f16_to_f32(uint32_t h16)
{
    return (float)__builtin_bit_cast(_Float16, (unsigned short)h16);
}

// float -> bf16 bits, round to nearest even; NaN stays a quiet NaN. Integer form, used where the exact bits are part
// of a stored format (quantizer scales).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f)
{
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// The same rounding in one instruction (gfx950 v_cvt_pk_bf16_f32, round to nearest even in the default mode; NaN
// becomes a quiet NaN), for output epilogues: no branch, so a store lane needs no exec-mask juggling.
__device__ __forceinline__ uint32_t f32_to_bf16_out(float f)
{
    return (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)f);
}

// Two e4m3fn bytes (byte pair HI of word w) -> two bf16, exact for every code, in one instruction: gfx950's
// v_cvt_scalef32_pk_bf16_fp8 (OCP e4m3) at scale 1.0. An e4m3 value has at most 4 significant bits and lies within
// bf16's normal range, subnormal codes (m 2^-9) included, so the conversion is exact; the two NaN codes give NaN.
// Checked on MI355X against the format's definition for all 256 codes in both byte pairs (also at scales 2^-10, 0.5,
// 2 and 2^10; the instruction takes only the scale's exponent: 1.5 acts as 1.0), and by every FP8 GPU parity test. It replaces
// v_cvt_pk_f32_fp8 + one v_perm_b32 of the two upper halves (3 -> 2 VALU per bf16 pair with its v_dot2).
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w)
{
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
}

// 8 bf16 weights (one 16-byte load) dot 8 x values.
__device__ __forceinline__ float dot_bf16_16B(const u32x4 w, const u32x4 x, float acc)
{
    acc = dot2_bf16(w.x, x.x, acc);
    acc = dot2_bf16(w.y, x.y, acc);
    acc = dot2_bf16(w.z, x.z, acc);
    acc = dot2_bf16(w.w, x.w, acc);
    return acc;
}

// 16 e4m3 weights (one 16-byte load) dot 16 x values (x0 = columns 0..7, x1 = columns 8..15).
__device__ __forceinline__ float fp8_word_dot(uint32_t w, uint32_t xa, uint32_t xb, float acc)
{
    acc = dot2_bf16(fp8x2_to_bf16x2<false>(w), xa, acc);
    acc = dot2_bf16(fp8x2_to_bf16x2<true>(w), xb, acc);
    return acc;
}
__device__ __forceinline__ float dot_fp8_16B(const u32x4 w, const u32x4 x0, const u32x4 x1, float acc)
{
    acc = fp8_word_dot(w.x, x0.x, x0.y, acc);
    acc = fp8_word_dot(w.y, x0.z, x0.w, acc);
    acc = fp8_word_dot(w.z, x1.x, x1.y, acc);
    acc = fp8_word_dot(w.w, x1.z, x1.w, acc);
    return acc;
}

// INT4: eight nibbles of one word (weights k..k+7, nibble j = weight k+j) against 8 x values staged in LDS in the
// order (x0,x2),(x4,x6),(x1,x3),(x5,x7). The even nibbles (one per byte, bits 0-3) and the odd ones (bits 4-7,
// shifted down) are masked into two words of four bytes; one v_perm_b32 per bf16 pair then places two of those bytes
// under a 0x43 high byte, giving bf16 (128 + q) (bf16 128.0 has an ulp of 1). So sum (128+q) x = sum q x + 128 sum x,
// and the caller removes the 128 sum x term (and the zero point) with the per-lane x sums. 7 VALU + 4 v_dot2 per
// 8 weights. c43 holds 0x43434343 (kept in a register: gfx9 VOP3 has no literal operand).
__device__ __forceinline__ float i4_word_dot(uint32_t w, const u32x4 x, float acc, uint32_t c43)
{
    const uint32_t lo = w & 0x0F0F0F0Fu;           // bytes: q0 q2 q4 q6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;    // bytes: q1 q3 q5 q7
    acc = dot2_bf16(__builtin_amdgcn_perm(c43, lo, 0x04010400u), x.x, acc);   // (128+q0, 128+q2)
    acc = dot2_bf16(__builtin_amdgcn_perm(c43, lo, 0x04030402u), x.y, acc);   // (128+q4, 128+q6)
    acc = dot2_bf16(__builtin_amdgcn_perm(c43, hi, 0x04010400u), x.z, acc);   // (128+q1, 128+q3)
    acc = dot2_bf16(__builtin_amdgcn_perm(c43, hi, 0x04030402u), x.w, acc);   // (128+q5, 128+q7)
    return acc;
}
// The same decode without the products: the four bf16 pairs (128 + q) of one word, in i4_word_dot's order, for
// callers that take several dot products per decoded word (one per activation row).
__device__ __forceinline__ void i4_word_decode(uint32_t w, uint32_t c43, uint32_t q4[4])
{
    const uint32_t lo = w & 0x0F0F0F0Fu;
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
    q4[0] = __builtin_amdgcn_perm(c43, lo, 0x04010400u);
    q4[1] = __builtin_amdgcn_perm(c43, lo, 0x04030402u);
    q4[2] = __builtin_amdgcn_perm(c43, hi, 0x04010400u);
    q4[3] = __builtin_amdgcn_perm(c43, hi, 0x04030402u);
}
__device__ __forceinline__ float dot_i4_16B(const u32x4 w, const u32x4 x0, const u32x4 x1, const u32x4 x2,
                                            const u32x4 x3, uint32_t c43)
{
    float d = i4_word_dot(w.x, x0, 0.0f, c43);
    d = i4_word_dot(w.y, x1, d, c43);
    d = i4_word_dot(w.z, x2, d, c43);
    d = i4_word_dot(w.w, x3, d, c43);
    return d;
}

// INT4 as bf16 subnormals (the decode of the kernels that stage x in LDS). Bits 0-7 of a bf16 whose high byte is 0
// hold any byte b as exactly b * 2^-133: b < 128 is the subnormal b * 2^-133, b >= 128 has exponent field 1 and
// mantissa b - 128, i.e. (1 + (b-128)/128) * 2^-126. So a nibble masked in place is q * 2^-133 in bits 0-3 and
// 16 q * 2^-133 in bits 4-7, and v_dot2_f32_bf16 takes subnormal operands as they are (measured on gfx950, as does
// the bf16 MFMA). With x staged as x * 2^a against bits 0-3 and x * 2^(a-4) against bits 4-7 every product is exactly
// q x 2^(a-133) (12 significant bits), so the dot of a word is 2^(a-133) sum q x with no offset to remove: 5 VALU (two
// masks, one shift, two masks) + 4 v_dot2 per 8 weights, where the 0x43-exponent decode takes 7 + 4 and leaves a
// 128 sum x term. The pairs are (q0,q4), (16q1,16q5), (q2,q6), (16q3,16q7) against x staged as
// (x0,x4)2^a, (x1,x5)2^(a-4), (x2,x6)2^a, (x3,x7)2^(a-4).
// The staging exponent a: 64 (the first scale, kI4StageFirst) when the activation row's largest |x| lies in
// [2^-20, 2^64), else one picked from that largest |x| (i4_stage_exp). Both keep every staged x finite, every sum far
// below 2^127 and the products normal down to at least 2^-37 times the largest |x| (2^-119 for the picked scale), far
// below fp32's 2^-24 resolution of the row's terms.
struct I4Stage {
    int a;      // x * 2^a staged against bits 0-3 (x * 2^(a-4) against bits 4-7)
    int unit;   // the dot products and lane sums come out in units of 2^unit, unit = a - 133
};
// From the largest bf16 magnitude pattern (sign cleared) of the row: exponent field e (0 for zero and subnormals
// counts as 1, inf/NaN as 254), largest |x| < 2^(e-126), a = 253 - e: the largest staged value lies in [2^126, 2^127).
__device__ __forceinline__ I4Stage i4_stage_exp(uint32_t max_abs_bits)
{
    int e = (int)(max_abs_bits >> 7);
    e = e < 1 ? 1 : (e > 254 ? 254 : e);
    return {253 - e, 120 - e};
}
constexpr I4Stage kI4StageFirst = {64, -69};
// the first scale's window as sign-cleared bf16 patterns: largest |x| >= 2^-20 (exponent field 107) and < 2^64 (191)
constexpr uint32_t kI4FirstLoBits = 107u << 7, kI4FirstHiBits = 191u << 7;

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u16x2 as_u16x2(uint32_t v) { return __builtin_bit_cast(u16x2, v); }
__device__ __forceinline__ uint32_t as_u32(u16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// The staged pairs of one x vector (8 bf16: x0..x7 in v.x..v.w, two per word), unscaled: (x0,x4), (x1,x5), (x2,x6),
// (x3,x7), one v_perm_b32 each.
__device__ __forceinline__ u32x4 i4_pairs(const u32x4 v)
{
    return {__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
            __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
}
// One pair at the first scale with integer operations: each nonzero bf16's exponent field raised by E (64 or 60),
// a packed 16-bit multiply-add of (|x| != 0) * (E << 7); zero stays zero. Exact for normal x below 2^64 (the window
// keeps the field <= 254); a subnormal x = m 2^-133 (|x| < 2^-126) is staged as (1 + m/128) 2^-127, an absolute
// error below 2^-126, under 2^-106 of the row's largest |x| in the window. `amax` collects the pair's |x| patterns.
// one16 holds 0x00010001 and e16 the pair (E << 7, E << 7), both opaque to the compiler (it would otherwise turn the
// packed minimum and multiply-add into a compare and select per half, or a shift and an add).
__device__ __forceinline__ uint32_t i4_scale_pair_first(uint32_t p, u16x2& amax, uint32_t one16, uint32_t e16)
{
    const u16x2 a = as_u16x2(p & 0x7FFF7FFFu);
    amax = __builtin_elementwise_max(amax, a);
    const u16x2 nz = __builtin_elementwise_min(a, as_u16x2(one16));
    return as_u32(nz * as_u16x2(e16) + as_u16x2(p));
}
// One pair scaled exactly by 2^a (v_ldexp_f32 per value, round trip through fp32; exact whenever the result stays a
// normal bf16, which the picked scale ensures for every |x| above 2^-119 times the row's largest).
__device__ __forceinline__ uint32_t i4_scale_pair_exact(uint32_t p, int a)
{
    const bf16x2 r = {(__bf16)__builtin_amdgcn_ldexpf(__uint_as_float(p << 16), a),
                      (__bf16)__builtin_amdgcn_ldexpf(__uint_as_float(p & 0xFFFF0000u), a)};
    return __builtin_bit_cast(uint32_t, r);
}
// The sum of a staged vector's 8 values in the decode's units: the staged pairs dotted with the decode of an all-ones
// word (q = 1: 2^-133 against the even pairs, 16 * 2^-133 against the odd ones), so the sum comes out exactly as the
// products of the hot loop do. c1 = 0x00010001 and c16 = 0x00100010 are held in registers.
__device__ __forceinline__ float i4_staged_sum(const u32x4 sx, uint32_t c1, uint32_t c16)
{
    float s = dot2_bf16(sx.x, c1, 0.0f);
    s = dot2_bf16(sx.y, c16, s);
    s = dot2_bf16(sx.z, c1, s);
    return dot2_bf16(sx.w, c16, s);
}
__device__ __forceinline__ float ldexp_f32(float v, int e) { return __builtin_amdgcn_ldexpf(v, e); }
__device__ __forceinline__ void i4_word_decode_dn(uint32_t w, uint32_t q4[4])
{
    const uint32_t t = w >> 8;
    q4[0] = w & 0x000F000Fu;   // (q0, q4)
    q4[1] = w & 0x00F000F0u;   // (16 q1, 16 q5)
    q4[2] = t & 0x000F000Fu;   // (q2, q6)
    q4[3] = t & 0x00F000F0u;   // (16 q3, 16 q7)
}
__device__ __forceinline__ float i4dn_word_dot(uint32_t w, const u32x4 x, float acc)
{
    uint32_t q4[4];
    i4_word_decode_dn(w, q4);
    acc = dot2_bf16(q4[0], x.x, acc);
    acc = dot2_bf16(q4[1], x.y, acc);
    acc = dot2_bf16(q4[2], x.z, acc);
    acc = dot2_bf16(q4[3], x.w, acc);
    return acc;
}
__device__ __forceinline__ float dot_i4dn_16B(const u32x4 w, const u32x4 x0, const u32x4 x1, const u32x4 x2,
                                              const u32x4 x3)
{
    float d = i4dn_word_dot(w.x, x0, 0.0f);
    d = i4dn_word_dot(w.y, x1, d);
    d = i4dn_word_dot(w.z, x2, d);
    d = i4dn_word_dot(w.w, x3, d);
    return d;
}

// Two floats -> one bf16 pair (v_cvt_pk_bf16_f32, round to nearest even).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi)
{
    const bf16x2 r = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, r);
}

// ---------------------------------------------------------------------------------------------------------------
// wave64 reduction with DPP adds: quad sums, row (16-lane) sums by rotation, then the gfx9 row broadcasts carry row 0
// into row 1 and rows 0-1 into rows 2-3, so lane 63 ends with the wave's total. The DPP move's old value is 0 (the
// identity of the add) for lanes outside the row mask, which lets the backend fuse each move into its v_add_f32:
// 6 DPP adds + 1 readlane. The order of additions is fixed, so results are bitwise reproducible.
// ---------------------------------------------------------------------------------------------------------------
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v)
{
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float v)
{
    v = dpp_add<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v = dpp_add<0x124, 0xF>(v);   // row_ror:4
    v = dpp_add<0x128, 0xF>(v);   // row_ror:8  -> every lane holds its row's sum
    v = dpp_add<0x142, 0xA>(v);   // row_bcast:15 into rows 1, 3
    v = dpp_add<0x143, 0xC>(v);   // row_bcast:31 into rows 2, 3 -> lane 63 holds the total
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// Two wave sums at once: v_permlane32_swap pairs the upper half of a with the lower half of b, so one add leaves
// half-sums of a in lanes 0-31 and of b in lanes 32-63; four DPP adds make 16-lane row sums and row_bcast:15 adds
// row 0 into row 1 and row 2 into row 3. Lane 31 ends with sum(a), lane 63 with sum(b): 7 VALU for two rows where
// wave_sum takes 12 and two readlanes. Fixed order, so bitwise reproducible.
__device__ __forceinline__ float wave_sum2(float a, float b)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    float v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    v = dpp_add<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v = dpp_add<0x124, 0xF>(v);   // row_ror:4
    v = dpp_add<0x128, 0xF>(v);   // row_ror:8
    v = dpp_add<0x142, 0xA>(v);   // row_bcast:15 into rows 1, 3
    return v;
}

// Wave maximum of non-negative values (0, the identity, fills lanes outside a DPP row mask): same steps as wave_sum,
// lane 63 ends with the maximum.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_max(uint32_t v)
{
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, false);
    return v > o ? v : o;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    v = dpp_max<0xB1, 0xF>(v);
    v = dpp_max<0x4E, 0xF>(v);
    v = dpp_max<0x124, 0xF>(v);
    v = dpp_max<0x128, 0xF>(v);
    v = dpp_max<0x142, 0xA>(v);
    v = dpp_max<0x143, 0xC>(v);
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over the 4 lanes of a quad (result in every lane of the quad).
__device__ __forceinline__ float quad_sum(float v)
{
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    return v;
}

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

}  // namespace paia
