"""GPU dequantisation must be bit-exact against the oracle ("Dequantised weights must be
bit-exact"), and the torch ops must give the C ABI's bits."""
import numpy as np
import pytest
import torch

from gpu_util import bits16, make, note
from paia_bench.inputs import to_device

pytestmark = pytest.mark.gpu


def f32_bits(t):
    return t.detach().cpu().contiguous().numpy().view(np.uint32)


def assert_same_floats(got, want, what):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ"
    bad = np.nonzero(got[~gn].view(np.uint32) != want[~wn].view(np.uint32))[0]
    assert bad.size == 0, f"{what}: {bad.size} values differ"


def test_dequant_fp8_every_code_bitexact(oracle, gemv_lib, cuda):
    """All 256 e4m3 codes (incl. subnormals, +-0, +-448 and the NaN codes) times several scales."""
    codes = np.tile(np.arange(256, dtype=np.uint8), (6, 1))
    scale = np.float32([1.0, 0.0125, 3.0e-3, 1.7e-7, 2.5, 1.0 / 448])
    Wq = torch.from_numpy(codes).to(cuda)
    s = torch.from_numpy(scale).to(cuda)
    out = torch.empty(6, 256, dtype=torch.float32, device=cuda)
    note("dequant fp8 all codes")
    gemv_lib.dequant_fp8(Wq.data_ptr(), s.data_ptr(), out.data_ptr(), 6, 256)
    torch.cuda.synchronize()
    assert_same_floats(out.cpu().numpy(), oracle.dequant_fp8(codes, scale), "fp8 all codes")


@pytest.mark.parametrize("fmt", ["fp8", "int4", "int4zp"])
def test_dequant_bitexact_seeded(oracle, gemv_lib, cuda, fmt):
    shapes = [(1, 128), (3, 384), (33, 2176), (1000, 3584), (4096, 4096), (3584, 18944)]
    for N, K in shapes:
        ops, np_ops = make(fmt, N, K)
        dev = to_device(ops, cuda)
        out = torch.empty(N, K, dtype=torch.float32, device=cuda)
        note(f"dequant {fmt} N={N} K={K}")
        if fmt == "fp8":
            gemv_lib.dequant_fp8(dev["Wq"].data_ptr(), dev["scale"].data_ptr(), out.data_ptr(), N, K)
            want = oracle.dequant_fp8(np_ops["Wq"], np_ops["scale"])
        elif fmt == "int4":
            gemv_lib.dequant_int4(dev["Wq"].data_ptr(), dev["scales"].data_ptr(), out.data_ptr(), N, K)
            want = oracle.dequant_int4(np_ops["Wq"], np_ops["scales"])
        else:
            gemv_lib.dequant_int4_zp(dev["Wq"].data_ptr(), dev["scales"].data_ptr(), dev["zeros"].data_ptr(),
                                     out.data_ptr(), N, K)
            want = oracle.dequant_int4_zp(np_ops["Wq"], np_ops["scales"], np_ops["zeros"])
        torch.cuda.synchronize()
        assert_same_floats(out.cpu().numpy(), want, f"{fmt} {N}x{K}")


def test_dequant_int4zp_odd_group_count(oracle, gemv_lib, cuda):
    """G odd (K = 384, 640): the last zero byte holds one group in its low nibble."""
    for N, K in [(5, 384), (17, 640)]:
        ops, np_ops = make("int4zp", N, K)
        dev = to_device(ops, cuda)
        out = torch.empty(N, K, dtype=torch.float32, device=cuda)
        gemv_lib.dequant_int4_zp(dev["Wq"].data_ptr(), dev["scales"].data_ptr(), dev["zeros"].data_ptr(),
                                 out.data_ptr(), N, K)
        torch.cuda.synchronize()
        assert_same_floats(out.cpu().numpy(), oracle.dequant_int4_zp(np_ops["Wq"], np_ops["scales"], np_ops["zeros"]),
                           f"zp odd G {N}x{K}")


def test_torch_ops_match_c_abi(oracle, gemv_lib, cuda):
    """torch.ops.paia_gemv.* produce the C ABI's bits; *_out writes in place; int32-packed INT4 is accepted."""
    from gpu_util import run_gemv
    from paia_gemv import ops as pops
    for fmt, (N, K) in [("bf16", (1000, 3584)), ("fp8", (4097, 4096)), ("int4", (513, 14336)),
                        ("int4zp", (4608, 3584))]:
        o, _ = make(fmt, N, K, bias=fmt in ("bf16", "fp8", "int4zp"))
        d = to_device(o, cuda)
        kind = fmt
        vid = gemv_lib.pick_variant(kind, N, K)
        note(f"torch op {fmt}")
        want = bits16(run_gemv(gemv_lib, fmt, d, vid))
        x2 = d["x"].view(1, K)
        if fmt == "bf16":
            y = pops.gemv_bf16(d["W"], x2, d["bias"])
        elif fmt == "fp8":
            y = pops.gemv_fp8(d["Wq"], d["scale"], x2, d["bias"])
        elif fmt == "int4":
            y = pops.gemv_int4(d["Wq"].view(torch.int32), d["scales"].view(torch.float16), x2)
        else:
            y = torch.empty(N, dtype=torch.bfloat16, device=cuda)
            pops.gemv_int4_zp(d["Wq"].view(torch.int32), d["scales"], d["zeros"], d["x"], d["bias"], out=y)
        assert np.array_equal(bits16(y), want), fmt
    o, np_ops = make("fp8", 64, 512)
    d = to_device(o, cuda)
    assert_same_floats(pops.dequant_fp8(d["Wq"], d["scale"]).cpu().numpy(),
                       oracle.dequant_fp8(np_ops["Wq"], np_ops["scale"]), "op dequant_fp8")
    with pytest.raises(RuntimeError):
        pops.gemv_bf16(torch.zeros(4, 12, dtype=torch.bfloat16, device=cuda),
                       torch.zeros(12, dtype=torch.bfloat16, device=cuda))
