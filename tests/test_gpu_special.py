"""The reference's special operands on every variant of every format, through the C ABI.

src/tests/test_gemv_bf16.py:20-37,56-61 runs every variant at 1000x3584 on W ~ U(-0.02, 0.02), x ~ U(-0.5, 0.5)
with two special cases: "zeros" (W = 0) and "large" (W x 1e4 clamped to +-3e4, x x 100), gated by
max|y - ref| / max|ref| < 2e-2, or max|y| < 2e-2 where ref is all zero. Here the same operands are built for BF16
and quantised for FP8 and the reference INT4 format with the package's quantizers (paia_gemv.quant, the
src/paia_gemv/quant.py semantics); for the asymmetric INT4 format "zeros" means q = z in every group (random codes,
random scales: the dequantised weight is exactly 0 while the kernel's arithmetic is not trivial). The fp64 oracle is
the reference. Extra, beyond the reference's test:
  * BF16 and FP8 with all-zero weights must give exactly +0 in every row (every product is 0);
  * the INT4 kernels compute s * (sum (128+q) x - (128+z) sum x), a cancellation of two terms of size ~128 |sum x|:
    zero weights with |x| ~ 100 (x ~ 100 N(0,1)) must stay within the gate;
  * the naive and unfused INT4 controls and the small-batch pick (M = 2, 4, 16) see the same operands;
  * activations over a wide range of magnitudes, random signs: "wide" (|x| = 2^-50 .. 2^50), "bigx" (2^50 .. 2^63),
    "low" (2^-40 .. 2^-20), "tiny" (every |x| in 2^-120 .. 2^-55) and "huge" (2^60 .. 2^99, outputs still finite in
    bf16). The INT4 kernels that stage x read the nibbles as bf16 subnormals against x scaled by a power of two: 2^64
    when the row's largest |x| lies in [2^-20, 2^64) ("wide", "bigx" and "low" reach both ends of that window), else a
    power each block picks from that largest |x| ("tiny", "huge": a fixed 2^64 would push the products into fp32
    subnormals or overflow x). The reference multiplies unscaled x in fp32 (src/paia_gemv/gemv_int4.cuh:33-52), so
    any finite x whose output is finite must pass its gate;
  * the same extreme activations on every row-streaming INT4 variant (M = 2..6), each activation row scaled by its
    own power of two so the rows of one call need different staging scales.
"""
import numpy as np
import pytest
import torch

from gpu_util import bits16, note, oracle_ref, run_gemv
from paia_bench.inputs import as_numpy, to_device
from paia_gemv import quant

pytestmark = pytest.mark.gpu

REF_GATE = 2e-2
N, K = 1000, 3584
N_TALL = 12288   # INT4 range cases also at this N: most variants' waves then make more than 4 weight loads
FORMATS = ["bf16", "fp8", "int4", "int4zp"]
# activation exponent ranges (|x| = m * 2^e, e uniform in [lo, hi])
EXP_RANGE = {"wide": (-50, 50), "bigx": (50, 63), "low": (-40, -20), "tiny": (-120, -55), "huge": (60, 99)}


def variants(lib, fmt):
    return {"bf16": lib.variants, "fp8": lib.variants_fp8}.get(fmt, lib.variants_int4)


def special_operands(fmt, special, seed=5, N=N):
    """CPU operands (torch tensors) of the reference's special cases for one format."""
    g = torch.Generator().manual_seed(seed)
    W = (torch.rand(N, K, generator=g) - 0.5) * 0.04
    x = torch.rand(K, generator=g) - 0.5
    if special == "zeros":
        W = torch.zeros_like(W)
    elif special == "large":
        W = (W.to(torch.bfloat16).float() * 1e4).clamp(-3e4, 3e4)
        x = x.to(torch.bfloat16).float() * 1e2
    elif special == "zeros_x100":       # zero weights, |x| ~ 100
        W = torch.zeros_like(W)
        x = torch.randn(K, generator=g) * 100.0
    elif special in EXP_RANGE:          # |x| = m * 2^e, m in [1, 2), random signs
        lo, hi = EXP_RANGE[special]
        e = torch.randint(lo, hi + 1, (K,), generator=g).double()
        sgn = torch.where(torch.rand(K, generator=g) < 0.5, -1.0, 1.0).double()
        x = (sgn * (1.0 + torch.rand(K, generator=g).double()) * torch.pow(2.0, e)).float()
    else:
        raise ValueError(special)
    o = {"fmt": fmt, "N": N, "K": K, "x": x.to(torch.bfloat16), "bias": None}
    if fmt == "bf16":
        o["W"] = W.to(torch.bfloat16)
    elif fmt == "fp8":
        o["Wq"], o["scale"] = quant.quantize_fp8_rowwise(W)
    elif fmt == "int4":
        o["Wq"], o["scales"] = quant.quantize_int4_g128(W)
    elif special.startswith("zeros"):
        G = K // 128
        z = torch.randint(0, 16, (N, G), generator=g, dtype=torch.uint8)
        q = z.repeat_interleave(128, dim=1)                       # q = z everywhere: every weight dequantises to 0
        s = (0.001 + 0.009 * torch.rand(N, G, generator=g)).to(torch.bfloat16)
        o["Wq"], o["scales"], o["zeros"] = quant.pack_int4(q), s, quant.pack_zeros(z)
    else:
        o["Wq"], o["scales"], o["zeros"] = quant.quantize_int4_zp_g128(W)
    return o


def gate(oracle, fmt, np_ops, yb, what):
    """NaN canary, then the reference's gate (src/tests/test_gemv_bf16.py:33-37) against the fp64 oracle."""
    assert not np.isnan(oracle.bf16_bits_to_f32(yb)).any(), f"{what}: unwritten rows"
    ref = np_ops["_ref"]
    _, _, rel = oracle.close_to_ref(yb, ref)
    assert rel < REF_GATE, f"{what}: {'max|y|' if not np.abs(ref).max() else 'rel err'} {rel:.3e}"
    return rel


def prepared(oracle, fmt, special, cuda, N=N):
    o = special_operands(fmt, special, N=N)
    np_ops = as_numpy(o)
    np_ops["_ref"] = oracle_ref(oracle, fmt, np_ops)
    return o, np_ops, to_device(o, cuda)


RANGES = ("wide", "bigx", "low", "tiny", "huge")
CASES = ([(f, sp, N) for f in FORMATS for sp in ("zeros", "large") + RANGES] +
         [(f, sp, N_TALL) for f in ("int4", "int4zp") for sp in RANGES] +
         [("int4", "zeros_x100", N), ("int4zp", "zeros_x100", N)])


@pytest.mark.parametrize("fmt,special,n", CASES)
def test_every_variant_on_special_operands(oracle, gemv_lib, cuda, fmt, special, n):
    o, np_ops, dev = prepared(oracle, fmt, special, cuda, N=n)
    worst = 0.0
    kinds = set()
    for v in variants(gemv_lib, fmt):
        kinds.add(gemv_lib.launch_kind(fmt, n, K, v["id"]))
        note(f"special {special} {fmt} {n}x{K} variant={v['id']}")
        yb = bits16(run_gemv(gemv_lib, fmt, dev, v["id"]))
        worst = max(worst, gate(oracle, fmt, np_ops, yb, f"{special} {fmt} {n}x{K} v{v}"))
        if special == "zeros" and fmt in ("bf16", "fp8"):
            assert np.all(yb == 0), f"{fmt} v{v}: zero weights must give +0 exactly"
    if fmt.startswith("int4") and special in RANGES:
        # both INT4 decodes of staged x are exercised: the subnormal one at both sizes, the 0x43 one (few weight loads
        # per wave) at the small one (either kernel with or without the drain)
        assert kinds & {"gemv_kernel", "gemv_kernel_dr"}, (fmt, n, kinds)
        assert n != N or kinds & {"gemv_kernel43", "gemv_kernel43_dr"}, (fmt, n, kinds)
    print(f"{special} {fmt} {n}x{K}: worst {worst:.2e} over {len(variants(gemv_lib, fmt))} variants, {sorted(kinds)}")


# (R, W) of the INT4 variants with 9, 12 or 14 waves per block (whole blocks per CU on the small shapes)
WHOLE_BLOCK_RW = {(1, 9), (2, 9), (1, 12), (1, 14)}


@pytest.mark.parametrize("fmt", ["int4", "int4zp"])
@pytest.mark.parametrize("special", ["wide", "tiny", "huge"])
def test_int4_whole_block_variants_on_the_subnormal_decode(oracle, gemv_lib, cuda, fmt, special):
    """The INT4 variants with 9, 12 or 14 waves per block at a height where their waves make more than 7 weight loads,
    so they run the subnormal decode, whose window flags are then folded over a wave count other than 4, 8 or 16: in
    the first scale's window (wide) and outside it, where the block stages x again (tiny, huge)."""
    n = 24576
    o, np_ops, dev = prepared(oracle, fmt, special, cuda, N=n)
    picked = [v for v in variants(gemv_lib, fmt) if (v["R"], v["W"]) in WHOLE_BLOCK_RW and v["H"] == 0]
    assert len(picked) == len(WHOLE_BLOCK_RW)
    for v in picked:
        assert gemv_lib.launch_kind(fmt, n, K, v["id"]) == "gemv_kernel", v
        note(f"whole-block variant {special} {fmt} {n}x{K} variant={v['id']}")
        yb = bits16(run_gemv(gemv_lib, fmt, dev, v["id"]))
        gate(oracle, fmt, np_ops, yb, f"{special} {fmt} {n}x{K} v{v}")


@pytest.mark.parametrize("special", ["zeros", "large", "zeros_x100"])
def test_int4_controls_on_special_operands(oracle, gemv_lib, cuda, special):
    """The naive (K1) control against the oracle; the unfused control against the bf16-rounded weights it uses."""
    o, np_ops, dev = prepared(oracle, "int4", special, cuda)
    note(f"special {special} naive")
    gate(oracle, "int4", np_ops, bits16(run_gemv(gemv_lib, "int4", dev, 0, mode="naive")), f"{special} naive")
    scratch = torch.empty(N * K, dtype=torch.bfloat16, device=cuda)
    note(f"special {special} unfused")
    yb = bits16(run_gemv(gemv_lib, "int4", dev, 0, mode="unfused", scratch=scratch))
    wb = oracle.dequant_int4_bf16(np_ops["Wq"], np_ops["scales"])
    ref = oracle.gemv_bf16_f64(wb, np_ops["x"])
    _, _, rel = oracle.close_to_ref(yb, ref)
    assert rel < REF_GATE, (special, rel)


@pytest.mark.parametrize("special", ["zeros", "large"])
@pytest.mark.parametrize("fmt", FORMATS)
def test_batch_pick_on_special_operands(oracle, gemv_lib, cuda, fmt, special):
    """The small-batch entry points at the library's pick, M = 2, 4, 16, every activation row the special x times a
    per-row factor (so rows differ), each row gated against the oracle."""
    o, np_ops, dev = prepared(oracle, fmt, special, cuda)
    L = gemv_lib
    for M in (2, 4, 16):
        f = torch.linspace(1.0, -1.0, M)
        xs = (o["x"].float()[None, :] * f[:, None]).to(torch.bfloat16)
        xd = xs.to(cuda)
        y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=cuda)
        v = L.batch_pick_variant(fmt, M, N, K)
        note(f"special batch {special} {fmt} M={M} variant={v}")
        if fmt == "bf16":
            L.batch_bf16(dev["W"].data_ptr(), xd.data_ptr(), None, y.data_ptr(), M, N, K, v)
        elif fmt == "fp8":
            L.batch_fp8(dev["Wq"].data_ptr(), dev["scale"].data_ptr(), xd.data_ptr(), None, y.data_ptr(), M, N, K, v)
        elif fmt == "int4":
            L.batch_int4(dev["Wq"].data_ptr(), dev["scales"].data_ptr(), xd.data_ptr(), y.data_ptr(), M, N, K, v)
        else:
            L.batch_int4_zp(dev["Wq"].data_ptr(), dev["scales"].data_ptr(), dev["zeros"].data_ptr(), xd.data_ptr(),
                            None, y.data_ptr(), M, N, K, v)
        torch.cuda.synchronize()
        yb = bits16(y).reshape(M, N)
        xb = xs.view(torch.int16).numpy().view(np.uint16)
        for m in range(M):
            row_ops = dict(np_ops, x=np.ascontiguousarray(xb[m]))
            row_ops["_ref"] = oracle_ref(oracle, fmt, row_ops)
            gate(oracle, fmt, row_ops, yb[m].copy(), f"batch {special} {fmt} M={M} row {m}")


@pytest.mark.parametrize("special", ["tiny", "huge", "wide", "low"])
@pytest.mark.parametrize("fmt", ["int4", "int4zp"])
def test_int4_row_streaming_variants_on_extreme_x(oracle, gemv_lib, cuda, fmt, special):
    """Every row-streaming INT4 variant (P = 0, M = 2..6) on the extreme activations, activation row m scaled by
    2^(5m) within the range's end (so the rows of one call stage x with different scales), each row gated against
    the fp64 oracle as the reference gates."""
    o, np_ops, dev = prepared(oracle, fmt, special, cuda)
    L = gemv_lib
    rows_vs = [v for v in L.variants_batch[fmt] if v["P"] == 0 and v["U"] != 0]
    assert rows_vs
    sign = -1.0 if special == "huge" else 1.0       # huge: scale down, so no row leaves the finite range
    worst = 0.0
    for v in rows_vs:
        M = v["X"]
        f = torch.tensor([2.0 ** (sign * 5 * m) for m in range(M)], dtype=torch.float64)
        xs = (o["x"].double()[None, :] * f[:, None]).to(torch.bfloat16)   # exact: powers of two
        xd = xs.to(cuda)
        y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=cuda)
        note(f"special rows {special} {fmt} M={M} variant={v}")
        if fmt == "int4":
            L.batch_int4(dev["Wq"].data_ptr(), dev["scales"].data_ptr(), xd.data_ptr(), y.data_ptr(), M, N, K,
                         v["id"])
        else:
            L.batch_int4_zp(dev["Wq"].data_ptr(), dev["scales"].data_ptr(), dev["zeros"].data_ptr(), xd.data_ptr(),
                            None, y.data_ptr(), M, N, K, v["id"])
        torch.cuda.synchronize()
        yb = bits16(y).reshape(M, N)
        xb = xs.view(torch.int16).numpy().view(np.uint16)
        for m in range(M):
            row_ops = dict(np_ops, x=np.ascontiguousarray(xb[m]))
            row_ops["_ref"] = oracle_ref(oracle, fmt, row_ops)
            worst = max(worst, gate(oracle, fmt, row_ops, yb[m].copy(), f"rows {special} {fmt} M={M} v{v} row {m}"))
    print(f"rows {special} {fmt}: worst {worst:.2e} over {len(rows_vs)} variants")
