"""The number facts the INT4 kernels' subnormal decode rests on, checked on the CPU with IEEE arithmetic.

The M = 1 kernel with x staged in LDS (paia-project_amd/csrc/gemv_device.h, i4_word_decode_dn; gemv_kernel.h,
i4_stage_x) reads a packed INT4 word w (nibble j = weight j, low nibble first, the reference's packing,
src/paia_gemv/quant.py) as four bf16 pairs by masking in place:

    (w & 0x000F000F), (w & 0x00F000F0), ((w >> 8) & 0x000F000F), ((w >> 8) & 0x00F000F0)

and takes their dot products against x staged as (x0,x4) 2^64, (x1,x5) 2^60, (x2,x6) 2^64, (x3,x7) 2^60, claiming the
sum is exactly 2^-69 sum_j q_j x_j. That needs (a) every byte b in bits 0-7 of a bf16 with a zero high byte to be
b * 2^-133 exactly, and (b) the masks and x order to pair every nibble with its own column. Both are checked here
against the plain nibble arithmetic (q_j = (w >> 4j) & 15) in float64; a wrong mask, shift, pair order or scale
fails (c) below. That the GPU's v_dot2_f32_bf16 and MFMA take subnormal bf16 operands as they are is a hardware fact
that the GPU parity tests (tests/test_gpu_*.py) exercise on every INT4 variant.
"""
import numpy as np

MASKS = (0x000F000F, 0x00F000F0)


def bf16_bits_to_f64(bits):
    """bf16 bit patterns (uint16/uint32 array) -> float64, through float32 (bf16 is the high half of a float32)."""
    return (np.asarray(bits, dtype=np.uint32) << np.uint32(16)).view(np.float32).astype(np.float64)


def to_bf16_bits(v):
    """float64 values that are exactly representable in bf16 -> their bf16 bits (asserts exactness)."""
    f = np.asarray(v, dtype=np.float32)
    bits = (f.view(np.uint32) >> np.uint32(16)).astype(np.uint32)
    assert np.array_equal(bf16_bits_to_f64(bits), f.astype(np.float64)), "value not exact in bf16"
    return bits


def test_every_low_byte_is_that_byte_times_2_pow_minus_133():
    b = np.arange(256, dtype=np.uint32)
    assert np.array_equal(bf16_bits_to_f64(b), b.astype(np.float64) * 2.0 ** -133)
    # b < 128: subnormal (exponent field 0); b >= 128: exponent field 1
    assert np.all(((b >> 7) & 1) == (b >= 128))


def decode_pairs(w):
    """The kernel's four masked pairs of each word, as (lo, hi) bf16 values in float64: shape [n, 4, 2]."""
    w = np.asarray(w, dtype=np.uint32)
    t = w >> np.uint32(8)
    words = [w & np.uint32(MASKS[0]), w & np.uint32(MASKS[1]), t & np.uint32(MASKS[0]), t & np.uint32(MASKS[1])]
    out = np.empty((w.size, 4, 2))
    for i, d in enumerate(words):
        out[:, i, 0] = bf16_bits_to_f64(d & np.uint32(0xFFFF))
        out[:, i, 1] = bf16_bits_to_f64(d >> np.uint32(16))
    return out


def staged_x(x):
    """x [n, 8] (bf16-exact float64) -> the staged pairs [n, 4, 2] as bf16 values, scaled as the kernel stages them."""
    order = [(0, 4, 2.0 ** 64), (1, 5, 2.0 ** 60), (2, 6, 2.0 ** 64), (3, 7, 2.0 ** 60)]
    out = np.empty((x.shape[0], 4, 2))
    for i, (a, b, s) in enumerate(order):
        for h, col in enumerate((a, b)):
            v = x[:, col] * s
            out[:, i, h] = bf16_bits_to_f64(to_bf16_bits(v))   # exact: a power-of-two scale of a bf16
    return out


def test_masks_give_each_nibble_its_own_scale():
    rng = np.random.default_rng(1)
    w = np.concatenate([rng.integers(0, 2 ** 32, 4096, dtype=np.uint64).astype(np.uint32),
                        np.array([0, 0xFFFFFFFF, 0x88888888, 0x0F0F0F0F, 0xF0F0F0F0, 0x12345678], dtype=np.uint32)])
    q = np.stack([(w >> np.uint32(4 * j)) & np.uint32(15) for j in range(8)], axis=1).astype(np.float64)
    d = decode_pairs(w) / 2.0 ** -133
    want = np.stack([q[:, [0, 4]], 16 * q[:, [1, 5]], q[:, [2, 6]], 16 * q[:, [3, 7]]], axis=1)
    assert np.array_equal(d, want)


def test_decoded_dot_is_2_pow_minus_69_times_the_nibble_dot():
    rng = np.random.default_rng(2)
    n = 4096
    w = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    # bf16-exact x over a wide range of magnitudes, signs and zeros
    x = rng.standard_normal((n, 8)) * np.exp2(rng.integers(-40, 40, (n, 1)))
    x[rng.random((n, 8)) < 0.05] = 0.0
    x = _round_bf16(x)
    q = np.stack([(w >> np.uint32(4 * j)) & np.uint32(15) for j in range(8)], axis=1).astype(np.float64)
    got = np.sum(decode_pairs(w) * staged_x(x), axis=(1, 2))      # every product exact in float64 (12 bits)
    want = 2.0 ** -69 * np.sum(q * x, axis=1)
    mag = 2.0 ** -69 * np.sum(np.abs(q * x), axis=1)              # float64 summation error is relative to this
    assert np.all(np.abs(got - want) <= 1e-15 * mag)
    # the zero-point form: (sum q x - z sum x), with the x sum in the same 2^-69 units, scaled back by 2^69, is
    # sum (q - z) x
    z = rng.integers(0, 16, n).astype(np.float64)
    sx = 2.0 ** -69 * x.sum(axis=1)
    ref = np.sum((q - z[:, None]) * x, axis=1)
    mag2 = np.sum(np.abs(q * x), axis=1) + z * np.sum(np.abs(x), axis=1)
    assert np.all(np.abs(2.0 ** 69 * (got - z * sx) - ref) <= 1e-14 * mag2)


def _round_bf16(x):
    """float64 -> nearest bf16 value (round to nearest even on the float32 bits), as float64 bits for to_bf16_bits."""
    f = np.asarray(x, dtype=np.float32).view(np.uint32)
    r = ((f + np.uint32(0x7FFF) + ((f >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)) << np.uint32(16)
    return r.view(np.float32).astype(np.float64)
