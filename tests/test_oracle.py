"""Pins the CPU oracle (oracle/paia_oracle.c) before anything is checked against it.

Each check is chosen so that a plausible mistake in the restatement (a dropped term, a wrong bias/shift, a wrong
rounding direction, a transposed nibble) fails at least one of them:
  * the reference's own known answers and exhaustive sweeps (src/tests/quant_host_selftest.cpp:11-44);
  * library routines that realise the same definitions (numpy float16, torch float8_e4m3fn and bfloat16);
  * golden vectors written by the reference's own quant_host.h (tests/golden/quant_host_vectors.npz);
  * the reference itself, compiled in place (oracle/_ref), where it was built;
  * closed forms and brute force for what none of those cover (asymmetric INT4, the GEMV references).
"""
import math
from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden" / "quant_host_vectors.npz"


def f32bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def same_floats(a, b):
    """Bitwise equality, with any NaN equal to any NaN."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and np.array_equal(f32bits(a[~na]), f32bits(b[~nb]))


# ---------------------------------------------------------------------------------------------------------------
# e4m3fn
# ---------------------------------------------------------------------------------------------------------------

def test_e4m3_known_answers(oracle):
    """quant_host_selftest.cpp:11-12."""
    L = oracle.lib()
    assert L.po_e4m3_to_f32(0x7E) == 448.0
    assert L.po_e4m3_to_f32(0x01) == 2.0 ** -9
    assert math.isnan(L.po_e4m3_to_f32(0x7F)) and math.isnan(L.po_e4m3_to_f32(0xFF))
    assert L.po_e4m3_to_f32(0x38) == 1.0
    assert L.po_e4m3_to_f32(0xB8) == -1.0
    assert L.po_e4m3_to_f32(0x08) == 2.0 ** -6          # smallest normal
    assert L.po_e4m3_to_f32(0x07) == 7 * 2.0 ** -9      # largest subnormal


def test_e4m3_decode_matches_torch_all_codes(oracle):
    """Library routine: torch float8_e4m3fn -> float32 for all 256 codes."""
    codes = torch.arange(256, dtype=torch.uint8)
    want = codes.view(torch.float8_e4m3fn).float().numpy()
    assert same_floats(oracle.e4m3_table(), want)


def test_e4m3_roundtrip_all_finite_codes(oracle):
    """quant_host_selftest.cpp:14: every finite code decodes and re-encodes to itself."""
    L = oracle.lib()
    for c in range(256):
        if (c & 0x7F) == 0x7F:
            continue
        assert L.po_f32_to_e4m3(L.po_e4m3_to_f32(c)) == c


def test_e4m3_encode_nearest_ties_even_bruteforce(oracle):
    """quant_host_selftest.cpp:16-23, with an independent brute force: nearest code by distance, ties to the code with
    an even mantissa lsb, after the +-448 clamp."""
    rng = np.random.default_rng(1)
    table = oracle.e4m3_table()[:127].astype(np.float64)           # codes 0..126, non-negative
    xs = np.concatenate([rng.uniform(-500, 500, 20000), rng.uniform(-0.5, 0.5, 10000) * 1e-3,
                         (table[:-1] + table[1:]) / 2]).astype(np.float32)
    got = oracle.e4m3_encode(xs)
    a = np.minimum(np.abs(xs.astype(np.float64)), 448.0)
    d = np.abs(a[:, None] - table[None, :])
    best = d.min(axis=1, keepdims=True)
    cand = d == best
    # among equally near codes, prefer an even code
    even = cand & (np.arange(127)[None, :] % 2 == 0)
    pick = np.where(even.any(axis=1), even.argmax(axis=1), cand.argmax(axis=1))
    assert np.array_equal(got & 0x7F, pick.astype(np.uint8))
    assert np.array_equal((got >> 7).astype(bool), np.signbit(xs))


def test_e4m3_encode_matches_torch(oracle):
    """Library routine: torch .clamp(+-448).to(float8_e4m3fn) is RNE-to-nearest (the quant.py:12 path)."""
    rng = np.random.default_rng(2)
    xs = np.concatenate([rng.uniform(-600, 600, 20000), rng.standard_normal(20000) * 0.05]).astype(np.float32)
    want = torch.from_numpy(xs).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(oracle.e4m3_encode(xs), want)


# ---------------------------------------------------------------------------------------------------------------
# fp16 / bf16
# ---------------------------------------------------------------------------------------------------------------

def test_f16_all_patterns_roundtrip(oracle):
    """quant_host_selftest.cpp:25: all 65536 patterns decode, and every non-NaN one re-encodes to itself; decode
    agrees with numpy's float16."""
    L = oracle.lib()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    dec = oracle.f16_bits_to_f32(h)
    assert same_floats(dec, h.view(np.float16).astype(np.float32))
    keep = ~np.isnan(dec)
    assert np.array_equal(oracle.f32_to_f16_bits(dec[keep]), h[keep])
    assert L.po_f32_to_f16(float("nan")) == 0x7E00


def test_f16_rne_matches_numpy(oracle):
    """Library routine: numpy float32 -> float16 (IEEE RNE, subnormals, overflow to inf), incl. exact ties."""
    rng = np.random.default_rng(3)
    mags = np.exp(rng.uniform(np.log(1e-9), np.log(1e5), 100000)).astype(np.float32)
    h = np.arange(0, 0x7BFF, dtype=np.uint16)
    ties = ((h.view(np.float16).astype(np.float64) + (h + 1).view(np.float16).astype(np.float64)) / 2)
    xs = np.concatenate([mags, -mags, ties.astype(np.float32), np.float32([65519.99, 65520, 1e30, 0.0, -0.0])])
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16_bits(xs), want)


def test_bf16_rne_matches_torch(oracle):
    """Library routine: torch float32 -> bfloat16 (RNE), incl. exact ties and NaN."""
    rng = np.random.default_rng(4)
    u = rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)
    u[:1000] = (u[:1000] & 0xFFFF0000) | 0x8000                    # exact ties
    xs = u.view(np.float32)
    want = torch.from_numpy(xs.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = oracle.f32_to_bf16_bits(xs)
    nan = np.isnan(xs)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7F80) == 0x7F80) and np.all((got[nan] & 0x7F) != 0)
    L = oracle.lib()
    for v in xs[:2000]:
        if not np.isnan(v):
            assert L.po_f32_to_bf16(float(v)) == oracle.f32_to_bf16_bits(np.float32([v]))[0]


# ---------------------------------------------------------------------------------------------------------------
# golden vectors from the reference's quant_host.h, and the reference itself where built
# ---------------------------------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def test_golden_formats(oracle, golden):
    assert same_floats(oracle.e4m3_table(), golden["e4m3_decode"])
    assert np.array_equal(oracle.e4m3_encode(golden["enc_in"]), golden["enc_out"])
    assert np.array_equal(oracle.f32_to_f16_bits(golden["f16_in"]), golden["f16_out"])


def test_golden_quantizers_and_dequant(oracle, golden):
    q, s = oracle.quantize_fp8_rowwise(golden["fp8_W"])
    assert np.array_equal(q, golden["fp8_q"]) and same_floats(s, golden["fp8_scale"])
    assert same_floats(oracle.dequant_fp8(q, s), golden["fp8_deq"])
    assert golden["fp8_scale"][2] == 1.0                            # zero row -> scale 1
    p, sc = oracle.quantize_int4_g128(golden["i4_W"])
    assert np.array_equal(p, golden["i4_packed"]) and np.array_equal(sc, golden["i4_scales"])
    assert same_floats(oracle.dequant_int4(p, sc), golden["i4_deq"])
    assert golden["i4_scales"][1, 1] == 0x3C00                      # zero group -> fp16 1.0
    assert golden["i4_scales"][3, 2] == 0                           # fp16 underflow stored as 0 ...
    assert np.all(np.concatenate([p[3, 128:192] & 0xF, p[3, 128:192] >> 4]) == 8)   # ... codes quantised with 1.0


def test_against_compiled_reference(oracle):
    """oracle/_ref: the reference's quant_host.h compiled in place (present where the checkout was at build time)."""
    R = oracle.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref not built here (reference checkout absent at build time)")
    rng = np.random.default_rng(5)
    for c in range(256):
        a, b = oracle.lib().po_e4m3_to_f32(c), R.ref_e4m3_decode(c)
        assert (math.isnan(a) and math.isnan(b)) or a == b
    xs = np.concatenate([rng.uniform(-500, 500, 5000), rng.standard_normal(5000) * 1e-3]).astype(np.float32)
    assert np.array_equal(oracle.e4m3_encode(xs), np.array([R.ref_e4m3_encode(float(v)) for v in xs], np.uint8))
    ys = (rng.standard_normal(5000) * np.exp(rng.uniform(-25, 11, 5000))).astype(np.float32)
    assert np.array_equal(oracle.f32_to_f16_bits(ys), np.array([R.ref_f32_to_f16_bits(float(v)) for v in ys], np.uint16))
    for N, K in [(3, 128), (7, 1152), (4, 3584)]:
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        q1, s1 = oracle.quantize_fp8_rowwise(W)
        q2, s2 = np.empty_like(q1), np.empty_like(s1)
        R.ref_quantize_fp8_rowwise(W, N, K, q2, s2)
        assert np.array_equal(q1, q2) and same_floats(s1, s2)
        p1, t1 = oracle.quantize_int4_g128(W)
        p2, t2 = np.empty_like(p1), np.empty_like(t1)
        R.ref_quantize_int4_g128(W, N, K, p2, t2)
        assert np.array_equal(p1, p2) and np.array_equal(t1, t2)


def test_reference_selftest_binary_passes():
    """The reference's own CPU self-test (src/tests/quant_host_selftest.cpp), built in place by oracle/Makefile."""
    import subprocess
    exe = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "quant_host_selftest"
    if not exe.exists():
        pytest.skip("oracle/_ref/quant_host_selftest not built here")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "passed" in r.stdout


# ---------------------------------------------------------------------------------------------------------------
# round-trip bounds and closed forms
# ---------------------------------------------------------------------------------------------------------------

def test_int4_roundtrip_bound(oracle):
    """quant_host_selftest.cpp:33-40: |deq - w| <= s/2 and nibbles in 1..15."""
    rng = np.random.default_rng(6)
    W = (rng.uniform(-0.5, 0.5, (5, 384)) * 1e-4).astype(np.float32)
    p, s = oracle.quantize_int4_g128(W)
    d = oracle.dequant_int4(p, s)
    sf = np.repeat(oracle.f16_bits_to_f32(s).reshape(s.shape), 128, axis=1)
    assert np.all(np.abs(d - W) <= 0.5 * sf * 1.0001 + 1e-12)
    nib = np.stack([p & 0xF, p >> 4], -1).reshape(W.shape)
    assert nib.min() >= 1 and nib.max() <= 15


def test_fp8_roundtrip_bound(oracle):
    """quant_host_selftest.cpp:42-44."""
    rng = np.random.default_rng(7)
    W = (rng.uniform(-0.5, 0.5, (5, 384)) * 1e-4).astype(np.float32)
    q, s = oracle.quantize_fp8_rowwise(W)
    d = oracle.dequant_fp8(q, s)
    assert np.all(np.abs(d - W) <= np.abs(W) * 0.0625 + s[:, None] * 2.0 ** -10)


def test_int4_zp_dequant_closed_form(oracle):
    """Asymmetric INT4 has no reference code: pin (q - z) * s_bf16 against an fp64 computation (exact in fp32),
    with an odd group count so the last zero byte's high nibble is padding."""
    rng = np.random.default_rng(8)
    N, K = 6, 640
    G = K // 128
    q = rng.integers(0, 16, (N, K)).astype(np.uint8)
    z = rng.integers(0, 16, (N, G)).astype(np.uint8)
    s = oracle.f32_to_bf16_bits(rng.uniform(0.001, 0.01, (N, G)).astype(np.float32)).reshape(N, G)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    zp = np.zeros((N, (G + 1) // 2), np.uint8)
    for g in range(G):
        zp[:, g // 2] |= (z[:, g] << (4 * (g % 2))).astype(np.uint8)
    want = (q.astype(np.float64) - np.repeat(z, 128, 1)) * np.repeat(oracle.bf16_bits_to_f32(s).astype(np.float64), 128, 1)
    got = oracle.dequant_int4_zp(packed, s, zp)
    assert np.array_equal(got.astype(np.float64), want)
    # a transposed nibble order (high nibble first) must not pass this check
    swapped = ((packed >> 4) | (packed << 4)).astype(np.uint8)
    assert not np.array_equal(oracle.dequant_int4_zp(swapped, s, zp).astype(np.float64), want)


def test_int4_bf16_copy_is_rounded_dequant(oracle):
    rng = np.random.default_rng(9)
    W = (rng.standard_normal((3, 256)) * 0.02).astype(np.float32)
    p, s = oracle.quantize_int4_g128(W)
    assert np.array_equal(oracle.dequant_int4_bf16(p, s), oracle.f32_to_bf16_bits(oracle.dequant_int4(p, s)))


def test_gemv_references_closed_form(oracle):
    """fp64 references equal numpy's fp64 matmul of the same dequantised operands (up to fp64 summation order),
    bias included; the fused per-format references equal the dequant-then-dot path; row subsets index correctly."""
    rng = np.random.default_rng(10)
    N, K = 37, 1152
    x = oracle.f32_to_bf16_bits(rng.standard_normal(K).astype(np.float32))
    b = oracle.f32_to_bf16_bits((rng.standard_normal(N) * 0.02).astype(np.float32))
    xf = oracle.bf16_bits_to_f32(x).astype(np.float64)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    want = W.astype(np.float64) @ xf + oracle.bf16_bits_to_f32(b)
    assert np.allclose(oracle.gemv_f64(W, x, b), want, rtol=1e-12, atol=1e-12)
    assert np.allclose(oracle.gemv_f32_seq(W, x, b), want, rtol=1e-4, atol=1e-5)
    q, s = oracle.quantize_fp8_rowwise(W)
    assert np.allclose(oracle.gemv_fp8_f64(q, s, x, b), oracle.gemv_f64(oracle.dequant_fp8(q, s), x, b), rtol=1e-12)
    p, sc = oracle.quantize_int4_g128(W)
    assert np.allclose(oracle.gemv_int4_f64(p, sc, x), oracle.gemv_f64(oracle.dequant_int4(p, sc), x), rtol=1e-12)
    Wb = oracle.f32_to_bf16_bits(W)
    rows = np.array([36, 0, 17], np.int32)
    assert np.allclose(oracle.gemv_bf16_f64(Wb, x, None, rows),
                       oracle.bf16_bits_to_f32(Wb).astype(np.float64)[rows] @ xf, rtol=1e-12)
    # brute force on a tiny case, term by term
    y = oracle.gemv_f64(W[:2, :8].copy(), x[:8].copy())
    assert abs(y[1] - sum(float(W[1, k]) * float(xf[k]) for k in range(8))) < 1e-15


def test_close_to_ref_gate(oracle):
    """The BASELINE gate: within atol + rtol*|ref| after bf16 rounding, and the reference's max-relative gate."""
    ref = np.array([1.0, -2.0, 0.5, 100.0])
    y = oracle.f32_to_bf16_bits(np.float32([1.0, -2.0, 0.5, 100.0]))
    assert oracle.close_to_ref(y, ref)[0]
    y_bad = oracle.f32_to_bf16_bits(np.float32([1.0, -2.0, 0.5, 103.0]))
    ok, _, rel = oracle.close_to_ref(y_bad, ref)
    assert not ok and abs(rel - 0.03) < 1e-6


# ---------------------------------------------------------------------------------------------------------------
# asymmetric INT4 quantizer (no reference code): pinned by closed forms, not by restating it
# ---------------------------------------------------------------------------------------------------------------
def _zp_groups(oracle, p, s, z, G):
    q = np.stack([p & 0xF, p >> 4], axis=-1).reshape(p.shape[0], -1)
    zz = np.stack([z & 0xF, z >> 4], axis=-1).reshape(z.shape[0], -1)[:, :G]
    return q, zz, oracle.bf16_bits_to_f32(s).reshape(s.shape)


def test_int4_zp_quantizer_recovers_constructed_groups(oracle):
    """W built as (q - z) * s from bf16 s, z in 0..15 and codes that include 0 and 15 in every group is recovered
    exactly: then lo = -z s, hi = (15 - z) s, (hi - lo) / 15 = s exactly and rint(w / s) + z = q."""
    rng = np.random.default_rng(21)
    N, K = 9, 640
    G = K // 128
    q = rng.integers(0, 16, (N, K))
    q[:, 0::128], q[:, 1::128] = 0, 15
    z = rng.integers(0, 16, (N, G))
    sb = oracle.f32_to_bf16_bits(rng.uniform(1e-3, 1e-1, (N, G)).astype(np.float32))
    s = oracle.bf16_bits_to_f32(sb)
    W = ((q - np.repeat(z, 128, axis=1)) * np.repeat(s, 128, axis=1)).astype(np.float32)
    p2, s2, z2 = oracle.quantize_int4_zp_g128(W)
    q2, zz2, _ = _zp_groups(oracle, p2, s2, z2, G)
    assert np.array_equal(s2, sb) and np.array_equal(zz2, z) and np.array_equal(q2, q)


def test_int4_zp_quantizer_roundtrip_bound_and_specials(oracle):
    """Random groups: codes in 0..15 and |w - (q - z) s| <= s/2 (+ the bf16 rounding of s over 15 steps); an all-zero
    group gives s = 1, z = 0, q = 0; a one-sided group keeps 0 representable (lo <= 0 <= hi)."""
    rng = np.random.default_rng(22)
    N, K = 7, 3584
    G = K // 128
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    W[1, 256:384] = 0.0                                    # zero group
    W[2, 0:128] = np.abs(W[2, 0:128])                      # positive-only group
    p, sb, zp = oracle.quantize_int4_zp_g128(W)
    q, z, s = _zp_groups(oracle, p, sb, zp, G)
    deq = oracle.dequant_int4_zp(p, sb, zp)
    sr = np.repeat(s, 128, axis=1)
    assert np.all(np.abs(W - deq) <= sr * (0.5 + 15 * 2.0 ** -8) + 1e-12)
    assert s[1, 2] == 1.0 and z[1, 2] == 0 and np.all(q[1, 256:384] == 0)
    assert z[2, 0] == 0
    assert zp.shape == (N, G // 2)
    _, _, z3 = oracle.quantize_int4_zp_g128(W[:, :384])      # odd G = 3: the last byte's high nibble is padding 0
    assert z3.shape == (N, 2) and np.all((z3[:, 1] >> 4) == 0)


def test_int4_zp_quantizer_matches_torch_definition(oracle):
    """The C restatement and the package's vectorised torch definition (paia_gemv.quant) agree bit for bit."""
    import torch
    from paia_gemv import quant
    rng = np.random.default_rng(23)
    for N, K in [(5, 384), (64, 4096), (3, 18944)]:
        W = (rng.standard_normal((N, K)) * rng.uniform(1e-3, 1.0)).astype(np.float32)
        p1, s1, z1 = oracle.quantize_int4_zp_g128(W)
        p2, s2, z2 = quant.quantize_int4_zp_g128(torch.from_numpy(W))
        assert np.array_equal(p1, p2.numpy()) and np.array_equal(z1, z2.numpy())
        assert np.array_equal(s1, s2.view(torch.int16).numpy().view(np.uint16))
