"""GPU parity of the small-batch matrix-core kernels (paia_gemv_batch_*, M = 1..16) against the CPU oracle.

Bars: every output row m is checked like an M = 1 GEMV against the fp64 oracle and the fp32-matmul reference of the
same x row (rtol 1e-2 / atol 1e-2 after bf16 rounding, and the reference harness gate max|y-ref|/max|ref| < 2e-2,
paia-bench/bench/ops/ours_bf16.py:83-89); every element must be written (NaN-prefilled outputs). Exact properties
at full size: with x rows = unit vectors e_k the kernel returns bf16(deq(W[:, k])) bit for bit, and a row's result
does not depend on the other rows of the batch (same variant => same summation order), so y(M rows)[m] equals
y(x[m] alone) bitwise.
"""
import numpy as np
import pytest
import torch

from gpu_util import bits16, dequant_oracle, make, note
from paia_bench.inputs import to_device
from test_batch_emulation import plan, rows_lds_limit, runs

pytestmark = pytest.mark.gpu

RTOL = ATOL = 1e-2
REF_GATE = 2e-2

AWK = {
    "bf16": [(1, 8), (17, 264), (33, 1032), (129, 4104), (1000, 3584)],
    "fp8": [(1, 16), (17, 528), (33, 1552), (129, 4112), (1000, 3584)],
    "int4": [(1, 128), (17, 384), (33, 2176), (129, 4224), (1000, 3584)],
}
AWK["int4zp"] = AWK["int4"]
REAL = [(6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336), (4608, 3584), (3584, 3584), (37888, 3584),
        (3584, 18944)]


def x_rows(M, K, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g).to(torch.bfloat16)


def run_batch(lib, fmt, dev, x, variant=-1, y=None, bias=True):
    """One batch call on device operands; returns y bf16 [M, N] (NaN-prefilled)."""
    M, K = x.shape
    N = dev["N"]
    if y is None:
        y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=x.device)
    b = dev.get("bias") if bias else None
    bp = b.data_ptr() if b is not None else None
    if fmt == "bf16":
        lib.batch_bf16(dev["W"].data_ptr(), x.data_ptr(), bp, y.data_ptr(), M, N, K, variant)
    elif fmt == "fp8":
        lib.batch_fp8(dev["Wq"].data_ptr(), dev["scale"].data_ptr(), x.data_ptr(), bp, y.data_ptr(), M, N, K, variant)
    elif fmt == "int4":
        lib.batch_int4(dev["Wq"].data_ptr(), dev["scales"].data_ptr(), x.data_ptr(), y.data_ptr(), M, N, K, variant)
    else:
        lib.batch_int4_zp(dev["Wq"].data_ptr(), dev["scales"].data_ptr(), dev["zeros"].data_ptr(), x.data_ptr(), bp,
                          y.data_ptr(), M, N, K, variant)
    return y


def oracle_rows(O, fmt, np_ops, xb, rows=None):
    """Per activation row: (fp64 oracle, fp32-matmul reference). xb: uint16 bit patterns [M, K]."""
    b = np_ops.get("bias")
    Wd = dequant_oracle(O, fmt, np_ops)
    out = []
    for m in range(xb.shape[0]):
        x = np.ascontiguousarray(xb[m])
        if fmt == "bf16":
            r64 = O.gemv_bf16_f64(np_ops["W"], x, b, rows)
        elif fmt == "fp8":
            r64 = O.gemv_fp8_f64(np_ops["Wq"], np_ops["scale"], x, b, rows)
        elif fmt == "int4":
            r64 = O.gemv_int4_f64(np_ops["Wq"], np_ops["scales"], x, rows)
        else:
            r64 = O.gemv_int4_zp_f64(np_ops["Wq"], np_ops["scales"], np_ops["zeros"], x, b, rows)
        r32 = O.gemv_f32_matmul(Wd, x, b)
        out.append((r64, r32 if rows is None else r32[rows]))
    return out


def check_rows(O, y, refs, what, rows=None):
    yb = bits16(y).reshape(y.shape[0], -1)
    worst = 0.0
    for m, (r64, r32) in enumerate(refs):
        ym = yb[m] if rows is None else yb[m][rows]
        assert not np.isnan(O.bf16_bits_to_f32(ym)).any(), f"{what} row {m}: unwritten outputs (NaN canary)"
        ok, excess, _ = O.close_to_ref(ym, r32, RTOL, ATOL)
        _, _, rel = O.close_to_ref(ym, r64, RTOL, ATOL)
        assert ok, f"{what} row {m}: outside rtol/atol {RTOL} (worst excess {excess:.3e})"
        assert rel < REF_GATE, f"{what} row {m}: reference gate rel_err {rel:.3e}"
        worst = max(worst, rel)
    return worst


def xbits(x):
    return x.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int4", "int4zp"])
def test_every_variant_awkward_shapes(oracle, gemv_lib, cuda, fmt):
    """Every batch variant (all P, U, W, S) on shapes with N tails inside a tile, K tails inside a k-block (BF16/FP8)
    and single rows, at M = 5 (rows past M of the MFMA tile unused) and M = 16 (full tile, several LDS chunks)."""
    worst = 0.0
    for N, K in AWK[fmt]:
        ops, np_ops = make(fmt, N, K, bias=fmt != "int4")
        dev = to_device(ops, cuda)
        for M in (5, 16):
            x = x_rows(M, K, 3000 + M + N + K)
            refs = oracle_rows(oracle, fmt, np_ops, xbits(x))
            xd = x.to(cuda)
            for v in gemv_lib.variants_batch[fmt]:
                if not runs(fmt, M, N, K, v, rows_lds_limit()):
                    # S*M*U too large for the LDS chunk, or a row-streaming variant of another M: the entry point
                    # refuses it (-2) before launching
                    with pytest.raises(RuntimeError, match="returned -2"):
                        run_batch(gemv_lib, fmt, dev, xd, v["id"])
                    continue
                note(f"batch {fmt} M={M} N={N} K={K} variant={v}")
                y = run_batch(gemv_lib, fmt, dev, xd, v["id"])
                torch.cuda.synchronize()
                worst = max(worst, check_rows(oracle, y, refs, f"{fmt} M={M} {N}x{K} v{v}"))
    print(f"batch {fmt}: worst relative error {worst:.2e}")


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int4", "int4zp"])
def test_row_streaming_variants_awkward_shapes(oracle, gemv_lib, cuda, fmt):
    """Every row-streaming variant (P = 0) at the M it serves (2..6, BF16 and FP8 2..8), and the M = 1 GEMV entry at M = 1,
    on the awkward shapes (N tails inside a row group, K tails inside a chunk, single rows); other M, and shapes whose
    M copies of x exceed the LDS, must return -2."""
    worst = 0.0
    rows_vs = [v for v in gemv_lib.variants_batch[fmt] if v["P"] == 0]
    ms = (1, 2, 3, 4, 5, 6, 7, 8) if fmt in ("bf16", "fp8") else (1, 2, 3, 4, 5, 6)
    assert len(rows_vs) == 6 * (len(ms) - 1) + 1
    for N, K in AWK[fmt]:
        ops, np_ops = make(fmt, N, K, bias=fmt != "int4")
        dev = to_device(ops, cuda)
        for M in ms:
            x = x_rows(M, K, 3100 + M + N + K)
            refs = oracle_rows(oracle, fmt, np_ops, xbits(x))
            xd = x.to(cuda)
            for v in rows_vs:
                if not runs(fmt, M, N, K, v, rows_lds_limit()):
                    with pytest.raises(RuntimeError, match="returned -2"):
                        run_batch(gemv_lib, fmt, dev, xd, v["id"])
                    continue
                note(f"rows {fmt} M={M} N={N} K={K} variant={v}")
                y = run_batch(gemv_lib, fmt, dev, xd, v["id"])
                torch.cuda.synchronize()
                worst = max(worst, check_rows(oracle, y, refs, f"{fmt} M={M} {N}x{K} v{v}"))
    print(f"rows {fmt}: worst relative error {worst:.2e}")


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int4", "int4zp"])
def test_real_shapes_every_m_default_variant(oracle, gemv_lib, cuda, fmt):
    """The BASELINE projection shapes at M = 1, 2, 3, 4, 8, 16 with the library's pick; sampled rows for the big
    shapes (the oracle's fp64 pass stays within seconds)."""
    for N, K in REAL:
        ops, np_ops = make(fmt, N, K, bias=fmt != "int4")
        dev = to_device(ops, cuda)
        rows = np.unique(np.concatenate([np.arange(0, N, 97), [N - 1]])).astype(np.int64)
        for M in (1, 2, 3, 4, 8, 16):
            x = x_rows(M, K, 4000 + M + N + K)
            refs = oracle_rows(oracle, fmt, np_ops, xbits(x), rows)
            note(f"batch {fmt} M={M} N={N} K={K} pick={gemv_lib.batch_pick_variant(fmt, M, N, K)}")
            y = run_batch(gemv_lib, fmt, dev, x.to(cuda))
            torch.cuda.synchronize()
            assert not torch.isnan(y).any(), f"{fmt} M={M} {N}x{K}: unwritten outputs"
            check_rows(oracle, y, refs, f"{fmt} M={M} {N}x{K}", rows)


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int4", "int4zp"])
def test_rows_independent_and_deterministic(gemv_lib, cuda, fmt):
    """y(M = 16)[m] == y(x[m] alone) bitwise for every m, for a split-K and a non-split variant, and two runs agree."""
    N, K = 4096, 14336
    ops, _ = make(fmt, N, K, bias=fmt != "int4")
    dev = to_device(ops, cuda)
    x = x_rows(16, K, 77).to(cuda)
    vs = gemv_lib.variants_batch[fmt]
    picks = [next(v["id"] for v in vs if v["S"] == 1 and v["X"] == 0),
             next(v["id"] for v in vs if v["S"] == 4 and v["U"] == 2 and v["X"] == 0),
             next(v["id"] for v in vs if v["S"] == 8 and v["X"] == 1)]
    for vid in picks:
        note(f"batch rows-independent {fmt} variant={vs[vid]}")
        y16 = run_batch(gemv_lib, fmt, dev, x, vid)
        y16b = run_batch(gemv_lib, fmt, dev, x, vid)
        torch.cuda.synchronize()
        assert torch.equal(y16.view(torch.int16), y16b.view(torch.int16)), "two runs differ"
        for m in (0, 1, 7, 15):
            y1 = run_batch(gemv_lib, fmt, dev, x[m:m + 1].contiguous(), vid)
            torch.cuda.synchronize()
            assert torch.equal(y1[0].view(torch.int16), y16[m].view(torch.int16)), f"row {m} depends on the batch"


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int4", "int4zp"])
def test_unit_vectors_exact_full_size(oracle, gemv_lib, cuda, fmt):
    """x rows = e_k for 8 columns k spread over K (incl. both ends): row m of y is bf16(deq(W[:, k_m])) bit for bit,
    on the largest BASELINE shape of the format."""
    N, K = (37888, 3584) if fmt != "bf16" else (28672, 4096)
    ops, np_ops = make(fmt, N, K)
    dev = to_device(ops, cuda)
    Wd = dequant_oracle(oracle, fmt, np_ops)
    cols = [0, 1, 127, 128, K // 2 + 5, K - 129, K - 2, K - 1]
    x = torch.zeros(len(cols), K, dtype=torch.bfloat16)
    for m, k in enumerate(cols):
        x[m, k] = 1.0
    note(f"batch unit vectors {fmt} {N}x{K}")
    y = run_batch(gemv_lib, fmt, dev, x.to(cuda), bias=False)
    torch.cuda.synchronize()
    yb = bits16(y).reshape(len(cols), N)
    for m, k in enumerate(cols):
        want = oracle.f32_to_bf16_bits(np.ascontiguousarray(Wd[:, k]).astype(np.float32))
        assert np.array_equal(yb[m], want), f"{fmt} column {k}: {np.count_nonzero(yb[m] != want)} rows differ"


def test_torch_ops_route_rows_to_batch_kernels(gemv_lib, cuda):
    """torch.ops.paia_gemv with x [M, K] (M > 1) == the batch C ABI bitwise; [M, N] output; out= form allocates
    nothing new; x [1, K] still runs the M = 1 kernels."""
    from paia_gemv import ops
    N, K = 4608, 3584
    o, _ = make("int4zp", N, K, bias=True)
    d = to_device(o, cuda)
    x = x_rows(6, K, 5).to(cuda)
    note("torch ops batch int4zp")
    y = ops.gemv_int4_zp(d["Wq"], d["scales"], d["zeros"], x, bias=d["bias"])
    ref = run_batch(gemv_lib, "int4zp", d, x)
    torch.cuda.synchronize()
    assert y.shape == (6, N) and torch.equal(y.view(torch.int16), ref.view(torch.int16))
    out = torch.empty(6, N, dtype=torch.bfloat16, device=cuda)
    ops.gemv_int4_zp(d["Wq"], d["scales"], d["zeros"], x, bias=d["bias"], out=out)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    y1 = ops.gemv_int4_zp(d["Wq"], d["scales"], d["zeros"], x[:1].contiguous(), bias=d["bias"])
    torch.cuda.synchronize()
    assert y1.shape == (1, N)
    o8, _ = make("fp8", N, K, bias=True)
    d8 = to_device(o8, cuda)
    y8 = ops.gemv_fp8(d8["Wq"], d8["scale"], x, bias=d8["bias"])
    r8 = run_batch(gemv_lib, "fp8", d8, x)
    torch.cuda.synchronize()
    assert torch.equal(y8.view(torch.int16), r8.view(torch.int16))


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int4", "int4zp"])
def test_m1_runs_the_m1_gemv(gemv_lib, cuda, fmt):
    """At M = 1 the batch pick is the M = 1 GEMV entry (the last of the table): bitwise equal to the M = 1 entry
    point with its own pick, also into a y that is only 2-byte aligned (the batch contract; the BF16 M = 1 entry
    point asks for 16)."""
    L = gemv_lib
    for N, K in [(4096, 4096), (37888, 3584), (1000, 3584), (33, {"bf16": 1032, "fp8": 1040}.get(fmt, 2176))]:
        ops, _ = make(fmt, N, K, bias=fmt != "int4")
        dev = to_device(ops, cuda)
        x = x_rows(1, K, 5000 + N + K).to(cuda)
        assert L.batch_pick_variant(fmt, 1, N, K) == len(L.variants_batch[fmt]) - 1
        want = torch.full((N,), float("nan"), dtype=torch.bfloat16, device=cuda)
        v = L.pick_variant(fmt, N, K)
        b = dev.get("bias")
        bp = b.data_ptr() if b is not None else None
        note(f"batch M=1 route {fmt} {N}x{K} m1-variant={v}")
        if fmt == "bf16":
            L.bf16_bias(dev["W"].data_ptr(), x.data_ptr(), bp, want.data_ptr(), N, K, v)
        elif fmt == "fp8":
            L.fp8_bias(dev["Wq"].data_ptr(), dev["scale"].data_ptr(), x.data_ptr(), bp, want.data_ptr(), N, K, v)
        elif fmt == "int4":
            L.int4(dev["Wq"].data_ptr(), dev["scales"].data_ptr(), x.data_ptr(), want.data_ptr(), N, K, v)
        else:
            L.int4_zp(dev["Wq"].data_ptr(), dev["scales"].data_ptr(), dev["zeros"].data_ptr(), x.data_ptr(), bp,
                      want.data_ptr(), N, K, v)
        for off in (0, 1):                             # y at a 16-byte boundary, then 2 bytes past it
            buf = torch.full((N + 8,), float("nan"), dtype=torch.bfloat16, device=cuda)
            y = buf[off:off + N].view(1, N)
            run_batch(L, fmt, dev, x, y=y)
            torch.cuda.synchronize()
            assert torch.equal(y[0].view(torch.int16), want.view(torch.int16)), (fmt, N, K, off)
            assert torch.isnan(buf[off + N:]).all() and (off == 0 or torch.isnan(buf[:off]).all())


def test_graph_capture_replays_match_eager(gemv_lib, cuda):
    """A captured batch call (split-K variant) replayed several times, with eager work and syncs between replays,
    matches the eager result every time."""
    N, K = 4096, 4096
    o, _ = make("fp8", N, K)
    d = to_device(o, cuda)
    x = x_rows(4, K, 9).to(cuda)
    vid = next(v["id"] for v in gemv_lib.variants_batch["fp8"] if v["S"] == 4 and v["U"] == 2 and v["X"] == 0)
    eager = run_batch(gemv_lib, "fp8", d, x, vid)
    torch.cuda.synchronize()
    y = torch.empty_like(eager)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    note("batch graph capture fp8")
    with torch.cuda.graph(g, stream=s):
        gemv_lib.batch_fp8(d["Wq"].data_ptr(), d["scale"].data_ptr(), x.data_ptr(), None, y.data_ptr(), 4, N, K, vid,
                           torch.cuda.current_stream().cuda_stream)
    for i in range(4):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), eager.view(torch.int16)), f"replay {i}"
        run_batch(gemv_lib, "fp8", d, x, vid)
        torch.cuda.synchronize()


def test_contract_codes(gemv_lib, cuda):
    """Bad M / K / alignment return -2 before any launch; a bad variant returns -1."""
    N, K = 64, 256
    W = torch.zeros(N, K, dtype=torch.bfloat16, device=cuda)
    x = torch.zeros(17, K, dtype=torch.bfloat16, device=cuda)
    y = torch.zeros(17, N, dtype=torch.bfloat16, device=cuda)
    L = gemv_lib._lib
    assert L.paia_gemv_batch_bf16(W.data_ptr(), x.data_ptr(), None, y.data_ptr(), 17, N, K, -1, None) == -2
    assert L.paia_gemv_batch_bf16(W.data_ptr(), x.data_ptr(), None, y.data_ptr(), 0, N, K, -1, None) == -2
    assert L.paia_gemv_batch_bf16(W.data_ptr(), x.data_ptr(), None, y.data_ptr(), 2, N, K - 4, -1, None) == -2
    assert L.paia_gemv_batch_bf16(W.data_ptr(), x.data_ptr() + 2, None, y.data_ptr(), 2, N, K, -1, None) == -2
    assert L.paia_gemv_batch_bf16(W.data_ptr(), x.data_ptr(), None, y.data_ptr(), 2, N, K, 10 ** 6, None) == -1
    assert L.paia_gemv_batch_int4(W.data_ptr(), W.data_ptr(), x.data_ptr(), y.data_ptr(), 2, N, 192, -1, None) == -2
