"""CPU emulation of the kernels' in-register decode tricks (no GPU), pinned against the formats' definitions.

The gfx950 kernels (paia-project_amd/csrc/gemv_device.h) decode weights with integer bit operations and v_perm_b32
byte selects, then multiply with v_dot2 bf16 against x values that stage_x (gemv_kernel.h) pre-pairs in LDS. This file
emulates those exact steps in numpy and checks them against the mathematical definitions, the way the reference pins
its own decode tricks (src/tests/emulate_formats.py:56-67,128-133):
  * INT4: every nibble value in every position of a word decodes to bf16(128 + q), and the staged x pairing makes
    sum over the four dot2 products == sum_j (128 + q_j) x_j for the word's eight weights;
  * FP8: packing the upper halves of two v_cvt_pk_f32_fp8 results with selector 0x07060302 gives bf16 values equal to
    the e4m3fn decode for every code (e4m3 values need <= 4 significant bits, so the upper half is exact).
v_perm_b32 semantics (CDNA ISA): D.byte[i] = byte sel.byte[i] of the 8-byte value {src0, src1}, where selector values
0-3 pick bytes of src1 and 4-7 bytes of src0 (only these selector values are used).
"""
import numpy as np

from oracle import oracle as O


def v_perm(src0, src1, sel):
    src0 = np.asarray(src0, dtype=np.uint64)
    src1 = np.asarray(src1, dtype=np.uint64)
    both = (src0 << np.uint64(32)) | src1
    out = np.zeros_like(src1)
    for i in range(4):
        s = (sel >> (8 * i)) & 0xFF
        assert s <= 7
        byte = (both >> np.uint64(8 * s)) & np.uint64(0xFF)
        out |= byte << np.uint64(8 * i)
    return out.astype(np.uint32)


def bf16_pair(u32):
    u32 = np.asarray(u32, dtype=np.uint32)
    return (O.bf16_bits_to_f32((u32 & 0xFFFF).astype(np.uint16)),
            O.bf16_bits_to_f32((u32 >> 16).astype(np.uint16)))


C43 = 0x43434343


def i4_decode_pairs(w):
    """gemv_device.h i4_word_dot: the four bf16x2 operands made from one 32-bit word of eight nibbles."""
    w = np.asarray(w, dtype=np.uint32)
    lo = w & np.uint32(0x0F0F0F0F)
    hi = (w >> np.uint32(4)) & np.uint32(0x0F0F0F0F)
    return [v_perm(C43, lo, 0x04010400), v_perm(C43, lo, 0x04030402),
            v_perm(C43, hi, 0x04010400), v_perm(C43, hi, 0x04030402)]


def stage_pairs_int4(xv):
    """gemv_kernel.h stage_x (INT4): the 16-byte x vector (x0..x7 as 4 words of bf16 pairs) re-paired for the dots."""
    a = [np.uint32(v) for v in xv]
    return [(a[0] & 0xFFFF) | ((a[1] << 16) & 0xFFFFFFFF), (a[2] & 0xFFFF) | ((a[3] << 16) & 0xFFFFFFFF),
            (a[0] >> 16) | (a[1] & 0xFFFF0000), (a[2] >> 16) | (a[3] & 0xFFFF0000)]


def test_int4_every_nibble_every_position_decodes_to_128_plus_q():
    # word with nibble value q in position j and a different value in every other position
    for j in range(8):
        for q in range(16):
            others = [(q + 5 + 3 * i) % 16 for i in range(8)]
            others[j] = q
            w = sum(v << (4 * i) for i, v in enumerate(others))
            pairs = i4_decode_pairs(np.array([w], dtype=np.uint32))
            got = {}
            order = [(0, 2), (4, 6), (1, 3), (5, 7)]          # weight indices carried by (low, high) of each pair
            for (a, b), pr in zip(order, pairs):
                lo, hi = bf16_pair(pr)
                got[a], got[b] = float(lo[0]), float(hi[0])
            assert got == {i: 128.0 + others[i] for i in range(8)}, (j, q)


def test_int4_word_dot_equals_definition():
    """sum of the four dot2 products == sum_j (128 + q_j) x_j, exactly, for random words and bf16 x."""
    rng = np.random.default_rng(3)
    for _ in range(2000):
        w = np.uint32(rng.integers(0, 2 ** 32))
        xb = O.f32_to_bf16_bits(rng.standard_normal(8).astype(np.float32))      # x0..x7 as bf16 bits
        xv = [int(xb[2 * i]) | (int(xb[2 * i + 1]) << 16) for i in range(4)]
        xp = stage_pairs_int4(xv)
        wp = i4_decode_pairs(np.array([w], dtype=np.uint32))
        acc = 0.0
        for a, b in zip(wp, xp):
            wl, wh = bf16_pair(a)
            xl, xh = bf16_pair(np.array([b], dtype=np.uint32))
            acc += float(wl[0]) * float(xl[0]) + float(wh[0]) * float(xh[0])
        q = [(int(w) >> (4 * i)) & 0xF for i in range(8)]
        x = O.bf16_bits_to_f32(xb).astype(np.float64)
        want = sum((128.0 + q[i]) * x[i] for i in range(8))
        assert abs(acc - want) <= 1e-12 * max(1.0, abs(want)), (acc, want)


def test_fp8_every_code_exact_in_bf16():
    """The FP8 decode (v_cvt_scalef32_pk_bf16_fp8 at scale 1) writes each e4m3fn value as a bf16: exact only because
    every finite e4m3 value has at most 4 significant bits and lies within bf16's normal range (subnormal codes
    included), so bf16 rounding of the decoded value changes nothing; the two NaN codes stay NaN. (The instruction
    itself is checked on the GPU over all 256 codes through every FP8 variant.)"""
    f = O.e4m3_table().astype(np.float32)
    finite = ~np.isnan(f)
    assert (~finite).sum() == 2 and np.isnan(f[[0x7F, 0xFF]]).all()
    bf = O.bf16_bits_to_f32(O.f32_to_bf16_bits(f[finite]))
    assert np.array_equal(bf, f[finite])
    nz = np.abs(f[finite]) > 0
    assert np.abs(f[finite][nz]).min() == 2.0 ** -9 and np.abs(f[finite]).max() == 448.0   # far inside bf16's range


# ---------------------------------------------------------------------------------------------------------------
# wave reductions (gemv_device.h wave_sum / wave_sum2): lane-exact emulation of the DPP and permlane network
# ---------------------------------------------------------------------------------------------------------------
def dpp_add(v, ctrl, row_mask):
    """v + update_dpp(old=0, v, ctrl, row_mask): lanes of rows outside row_mask add 0."""
    v = np.asarray(v, dtype=np.float64)
    src = np.zeros(64)
    for i in range(64):
        row, j = divmod(i, 16)
        if ctrl == 0xB1:
            s = (i & ~3) | ((i & 3) ^ 1)
        elif ctrl == 0x4E:
            s = (i & ~3) | ((i & 3) ^ 2)
        elif ctrl in (0x124, 0x128):
            n = ctrl & 0xF
            s = row * 16 + (j - n) % 16
        elif ctrl == 0x142:          # row_bcast:15 -> lane 15 of the previous row
            s = (row - 1) * 16 + 15 if row > 0 else None
        elif ctrl == 0x143:          # row_bcast:31 -> lane 31
            s = 31 if row > 1 else None
        else:
            raise ValueError(ctrl)
        src[i] = v[s] if ((row_mask >> row) & 1) and s is not None else 0.0
    return v + src


def wave_sum_lanes(v):
    for ctrl, mask in [(0xB1, 0xF), (0x4E, 0xF), (0x124, 0xF), (0x128, 0xF), (0x142, 0xA), (0x143, 0xC)]:
        v = dpp_add(v, ctrl, mask)
    return v


def wave_sum2_lanes(a, b):
    """v_permlane32_swap(a, b): a keeps lanes 0-31 and takes b's lanes 0-31 in 32-63; b takes a's 32-63 in 0-31."""
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    a2 = np.concatenate([a[:32], b[:32]])
    b2 = np.concatenate([a[32:], b[32:]])
    v = a2 + b2
    for ctrl, mask in [(0xB1, 0xF), (0x4E, 0xF), (0x124, 0xF), (0x128, 0xF), (0x142, 0xA)]:
        v = dpp_add(v, ctrl, mask)
    return v


def test_wave_reductions_sum_every_lane_once():
    rng = np.random.default_rng(3)
    for _ in range(20):
        a = rng.integers(-1000, 1000, 64).astype(np.float64)
        b = rng.integers(-1000, 1000, 64).astype(np.float64)
        assert wave_sum_lanes(a)[63] == a.sum()
        v = wave_sum2_lanes(a, b)
        assert v[31] == a.sum() and v[63] == b.sum()
    # each lane's contribution counted exactly once (unit vectors)
    for i in range(64):
        e = np.zeros(64)
        e[i] = 1.0
        assert wave_sum_lanes(e)[63] == 1.0
        assert wave_sum2_lanes(e, 2 * e)[31] == 1.0 and wave_sum2_lanes(e, 2 * e)[63] == 2.0
