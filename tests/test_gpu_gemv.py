"""GPU parity of the fused GEMV kernels against the CPU oracle, through the C ABI.

Bars: outputs within rtol 1e-2 / atol 1e-2 of the fp32-accumulated reference after bf16
rounding, and the reference harness's gate max|y-ref|/max|ref| < 2e-2 against the fp64 oracle
(paia-bench/bench/ops/ours_bf16.py:83-89). Every output row must be written (NaN-prefilled outputs,
src/tests/test_gemv_bf16.py:30). At full BASELINE sizes a size-independent exact property is checked: with x = e_k
the kernel must return bf16(deq(W[:, k])) bit for bit in every row.
"""
import numpy as np
import pytest
import torch

from gpu_util import bits16, dequant_oracle, make, nan_filled, note, oracle_ref, run_gemv
from paia_bench.inputs import to_device

pytestmark = pytest.mark.gpu

RTOL = ATOL = 1e-2          # BASELINE gate, after bf16 rounding of the reference
REF_GATE = 2e-2             # reference harness gate: max|y - ref| / max|ref|

AWK = {
    "bf16": [(1, 8), (1, 256), (3, 264), (7, 520), (33, 1032), (129, 4104), (1000, 3584), (4097, 4096), (513, 14336)],
    "fp8": [(1, 16), (3, 528), (7, 1040), (33, 1552), (129, 4112), (1000, 3584), (4097, 4096), (513, 14336)],
    "int4": [(1, 128), (3, 384), (7, 1152), (33, 2176), (129, 4224), (1000, 3584), (4097, 4096), (513, 14336)],
}
AWK["int4zp"] = AWK["int4"]
REAL = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (3584, 3584), (512, 3584), (18944, 3584),
        (3584, 18944), (6144, 4096), (4608, 3584)]
BASELINE_SHAPES = [(6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336),
                   (4608, 3584), (3584, 3584), (37888, 3584), (3584, 18944)]


def variants(lib, fmt):
    return {"bf16": lib.variants, "fp8": lib.variants_fp8}.get(fmt, lib.variants_int4)


def refs(O, fmt, np_ops):
    """(fp64 oracle, fp32-matmul reference) for the operands."""
    if "_refs" not in np_ops:
        Wd = dequant_oracle(O, fmt, np_ops)
        np_ops["_refs"] = (oracle_ref(O, fmt, np_ops), O.gemv_f32_matmul(Wd, np_ops["x"], np_ops.get("bias")))
    return np_ops["_refs"]


def check(O, fmt, np_ops, y, what):
    yb = bits16(y)
    assert not np.isnan(O.bf16_bits_to_f32(yb)).any(), f"{what}: unwritten rows (NaN canary)"
    ref64, ref32 = refs(O, fmt, np_ops)
    ok, excess, _ = O.close_to_ref(yb, ref32, RTOL, ATOL)
    _, _, rel = O.close_to_ref(yb, ref64, RTOL, ATOL)
    assert ok, f"{what}: outside rtol/atol {RTOL} (worst excess {excess:.3e})"
    assert rel < REF_GATE, f"{what}: reference gate rel_err {rel:.3e}"
    return rel


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int4", "int4zp"])
def test_every_variant_on_awkward_shapes(oracle, gemv_lib, cuda, fmt):
    """All variants (as src/tests/test_gemv_bf16.py:94-100 and gemv_bf16_check.cu:367-380 do) on awkward shapes:
    K tails inside a chunk, N not a multiple of any tile, single rows."""
    worst = 0.0
    for N, K in AWK[fmt]:
        ops, np_ops = make(fmt, N, K)
        dev = to_device(ops, cuda)
        for v in variants(gemv_lib, fmt):
            note(f"{fmt} N={N} K={K} variant={v}")
            y = run_gemv(gemv_lib, fmt, dev, v["id"])
            torch.cuda.synchronize()
            worst = max(worst, check(oracle, fmt, np_ops, y, f"{fmt} {N}x{K} v{v}"))
    print(f"{fmt}: worst relative error {worst:.2e}")


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int4", "int4zp"])
def test_real_shapes_picked_and_default_variant(oracle, gemv_lib, cuda, fmt):
    """The library's per-shape variant and the harness default, on every real and BASELINE projection shape."""
    kmult = {"bf16": 8, "fp8": 16}.get(fmt, 128)
    kind = fmt
    default = {"bf16": (2, 4, 4, 0, 1), "fp8": (2, 2, 4, 0, 1)}.get(fmt, (4, 2, 4, 0, 1))
    vdef = next(v["id"] for v in variants(gemv_lib, fmt) if (v["R"], v["U"], v["W"], v["S"], v["H"]) == default)
    kinds = set()
    for N, K in sorted(set(REAL + BASELINE_SHAPES)):
        if K % kmult:
            continue
        ops, np_ops = make(fmt, N, K)
        dev = to_device(ops, cuda)
        for vid in sorted({gemv_lib.pick_variant(kind, N, K), vdef}):
            note(f"{fmt} N={N} K={K} variant={vid}")
            kinds.add(gemv_lib.launch_kind(fmt, N, K, vid))
            y = run_gemv(gemv_lib, fmt, dev, vid)
            torch.cuda.synchronize()
            check(oracle, fmt, np_ops, y, f"{fmt} {N}x{K} v{vid}")
    # both ends of the row-parallel walk ran: the plain loop (more than two items per wave) and the drain
    assert kinds & {"gemv_kernel", "gemv_kernel43"} and kinds & {"gemv_kernel_dr", "gemv_kernel43_dr"}, kinds


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int4zp"])
def test_bias_epilogue_qwen_qkv(oracle, gemv_lib, cuda, fmt):
    """Qwen2.5 qkv 4608x3584 with the bf16 bias epilogue: y = bf16(acc + bias), on every fifth
    variant and always on the library's own pick for the shape (what a caller of variant -1 gets)."""
    N, K = 4608, 3584
    ops, np_ops = make(fmt, N, K, bias=True)
    dev = to_device(ops, cuda)
    ids = sorted({v["id"] for v in variants(gemv_lib, fmt)[::5]} | {gemv_lib.pick_variant(fmt, N, K)})
    assert gemv_lib.pick_variant(fmt, N, K) in ids
    for vid in ids:
        note(f"bias {fmt} variant={vid}")
        y = run_gemv(gemv_lib, fmt, dev, vid)
        torch.cuda.synchronize()
        check(oracle, fmt, np_ops, y, f"bias {fmt} v{vid}")


# K whose staged x does not fit the 64 KiB of LDS (BF16/FP8 K > 32768, INT4 K > 30720; split-K variants earlier):
# the launch runs the x-from-global kernel whatever the variant. The reference accepts any K of the alignment rule
# (src/paia_gemv/gemv_bf16.cu:50-51, gemv_quant.cu:66,75).
BIG_K = {"bf16": [(33, 40000), (1, 65544), (64, 32768)], "fp8": [(129, 32784), (7, 100000)],
         "int4": [(65, 30848), (3, 65664)], "int4zp": [(65, 30848), (3, 65664)]}


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int4", "int4zp"])
def test_k_beyond_lds_staging(oracle, gemv_lib, cuda, fmt):
    """K beyond the LDS staging bound on the x-from-global kernel: the picked variant, a split-K and a row-parallel
    variant (all run it) against the oracle, with bias where the format takes one."""
    vs = variants(gemv_lib, fmt)
    h1 = next(v["id"] for v in vs if (v["R"], v["U"], v["W"], v["H"]) == (2, 2, 4, 1))
    h0 = next(v["id"] for v in vs if (v["R"], v["U"], v["W"], v["H"]) == (1, 1, 8, 0))
    for N, K in BIG_K[fmt]:
        ops, np_ops = make(fmt, N, K, bias=fmt != "int4")
        dev = to_device(ops, cuda)
        for vid in sorted({gemv_lib.pick_variant(fmt, N, K), h0, h1}):
            note(f"big K {fmt} N={N} K={K} variant={vid}")
            y = run_gemv(gemv_lib, fmt, dev, vid)
            torch.cuda.synchronize()
            check(oracle, fmt, np_ops, y, f"big K {fmt} {N}x{K} v{vid}")


def column_dequant(O, fmt, np_ops, k):
    """Exact dequantised column k (fp32 [N]) from the oracle, via a one-group / one-chunk slice."""
    if fmt == "bf16":
        return O.bf16_bits_to_f32(np_ops["W"][:, k].copy())
    if fmt == "fp8":
        k0 = k - k % 16
        return O.dequant_fp8(np_ops["Wq"][:, k0:k0 + 16].copy(), np_ops["scale"])[:, k % 16]
    g = k // 128
    pk = np_ops["Wq"][:, g * 64:(g + 1) * 64].copy()
    if fmt == "int4":
        return O.dequant_int4(pk, np_ops["scales"][:, g:g + 1].copy())[:, k % 128]
    z = (np_ops["zeros"][:, g // 2] >> (4 * (g % 2))) & 0xF
    return O.dequant_int4_zp(pk, np_ops["scales"][:, g:g + 1].copy(), z.astype(np.uint8)[:, None].copy())[:, k % 128]


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int4", "int4zp"])
def test_unit_vector_exact_full_size(oracle, gemv_lib, cuda, fmt):
    """Size-independent exact check at every BASELINE shape: x = e_k gives y = bf16(deq(W[:, k])) in every row
    (every row index, the chunk and group holding k, the K tail and the epilogue are all exercised)."""
    kind = fmt
    shapes = BASELINE_SHAPES + ([(128256, 4096)] if fmt == "bf16" else [])
    for N, K in shapes:
        ops, np_ops = make(fmt, N, K)
        dev = to_device(ops, cuda)
        vid = gemv_lib.pick_variant(kind, N, K)
        for k in sorted({0, 127, 128, 1000, K // 2 + 37, K - 129, K - 1}):
            note(f"unit {fmt} N={N} K={K} k={k} variant={vid}")
            x = torch.zeros(K, dtype=torch.bfloat16, device=cuda)
            x[k] = 1.0
            d = dict(dev, x=x)
            y = bits16(run_gemv(gemv_lib, fmt, d, vid))
            want = oracle.f32_to_bf16_bits(column_dequant(oracle, fmt, np_ops, k))
            # an e4m3 -0 weight (code 0x80) times 1, summed with the +0 products of the other columns, is +0 in
            # IEEE arithmetic (as in the fp64 oracle sum): compare zeros without their sign
            y = np.where((y & 0x7FFF) == 0, 0, y)
            want = np.where((want & 0x7FFF) == 0, 0, want)
            bad = np.nonzero(y != want)[0]
            assert bad.size == 0, f"{fmt} {N}x{K} k={k}: {bad.size} rows differ, first {bad[:5]}"


@pytest.mark.parametrize("N,K", [(512, 1024), (300, 3584)])
def test_fp8_every_code_every_variant_exact(oracle, gemv_lib, cuda, N, K):
    """Every finite e4m3 code (the 14 subnormal codes and both zeros included) through every FP8 variant and the
    batch picks, bit for bit: W[r, j] = code (r + j) mod 256, row scales 2^((r mod 9) - 4), and x = e_k give
    y[r] = bf16(deq(W[r, k]) * scale[r]) (exact: at most 4 significant bits times a power of two). The two NaN codes
    are replaced by zeros (0 * NaN in the other columns would make every row NaN); zeros are compared without their
    sign (-0 plus the other columns' +0 products is +0)."""
    codes = ((np.arange(N)[:, None] + np.arange(K)[None, :]) % 256).astype(np.uint8)
    codes[codes == 0x7F] = 0x00
    codes[codes == 0xFF] = 0x80
    scale = (2.0 ** ((np.arange(N) % 9) - 4)).astype(np.float32)
    dev = to_device({"fmt": "fp8", "N": N, "K": K, "Wq": torch.from_numpy(codes), "scale": torch.from_numpy(scale)},
                    cuda)

    def want_col(k):
        k0 = k - k % 16
        w = oracle.f32_to_bf16_bits(oracle.dequant_fp8(codes[:, k0:k0 + 16].copy(), scale)[:, k % 16])
        return np.where((w & 0x7FFF) == 0, 0, w)

    def zeroless(y):
        y = bits16(y)
        return np.where((y & 0x7FFF) == 0, 0, y)

    ks = sorted({0, 1, 127, 255, K // 2 + 3, K - 1})
    for k in ks:
        x = torch.zeros(K, dtype=torch.bfloat16, device=cuda)
        x[k] = 1.0
        want = want_col(k)
        d = dict(dev, x=x)
        for v in variants(gemv_lib, "fp8"):
            note(f"fp8 every code N={N} K={K} k={k} variant={v}")
            bad = np.nonzero(zeroless(run_gemv(gemv_lib, "fp8", d, v["id"])) != want)[0]
            assert bad.size == 0, f"fp8 {N}x{K} k={k} v{v}: {bad.size} rows differ, first {bad[:5]}"
    for M in (2, 5, 8, 16):
        kk = [ks[m % len(ks)] for m in range(M)]
        xm = torch.zeros(M, K, dtype=torch.bfloat16)
        for m, k in enumerate(kk):
            xm[m, k] = 1.0
        xm = xm.to(cuda)
        y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=cuda)
        note(f"fp8 every code batch M={M} N={N} K={K}")
        gemv_lib.batch_fp8(dev["Wq"].data_ptr(), dev["scale"].data_ptr(), xm.data_ptr(), None, y.data_ptr(), M, N, K,
                           -1)
        for m, k in enumerate(kk):
            bad = np.nonzero(zeroless(y[m]) != want_col(k))[0]
            assert bad.size == 0, f"fp8 batch M={M} {N}x{K} row {m} k={k}: {bad.size} rows differ, first {bad[:5]}"


def test_lm_head_bf16_sampled_rows(oracle, gemv_lib, cuda):
    """The bf16 lm_heads ([4]); fp64 check on sampled rows (gemv_bf16_check.cu:79-83)."""
    rng = np.random.default_rng(11)
    for N, K in [(152064, 3584), (128256, 4096)]:
        ops, np_ops = make("bf16", N, K)
        dev = to_device(ops, cuda)
        vid = gemv_lib.pick_variant("bf16", N, K)
        note(f"lm_head bf16 N={N} K={K} variant={vid}")
        y = bits16(run_gemv(gemv_lib, "bf16", dev, vid))
        assert not np.isnan(oracle.bf16_bits_to_f32(y)).any()
        rows = np.unique(np.concatenate([np.arange(8), N - 1 - np.arange(8), rng.integers(0, N, 256)])).astype(np.int32)
        ref = oracle.gemv_bf16_f64(np_ops["W"], np_ops["x"], None, rows)
        ok, excess, rel = oracle.close_to_ref(y[rows], ref, RTOL, ATOL)
        assert ok and rel < REF_GATE, (N, K, excess, rel)


def test_int4_naive_and_unfused_controls(oracle, gemv_lib, cuda):
    """K1 naive control against the fp64 oracle; the unfused control against the bf16-rounded-weight reference it
    computes (src/tests/gemv_bf16_check.cu:350-352)."""
    for N, K in AWK["int4"] + [(4096, 4096), (3584, 18944)]:
        ops, np_ops = make("int4", N, K)
        dev = to_device(ops, cuda)
        note(f"naive N={N} K={K}")
        y = run_gemv(gemv_lib, "int4", dev, 0, mode="naive")
        torch.cuda.synchronize()
        check(oracle, "int4", np_ops, y, f"naive {N}x{K}")
        scratch = torch.empty(N * K, dtype=torch.bfloat16, device=cuda)
        note(f"unfused N={N} K={K}")
        y = bits16(run_gemv(gemv_lib, "int4", dev, 0, mode="unfused", scratch=scratch))
        torch.cuda.synchronize()
        wb = oracle.dequant_int4_bf16(np_ops["Wq"], np_ops["scales"])
        assert np.array_equal(bits16(scratch).reshape(N, K), wb), "unfused scratch must be bf16_rn(deq)"
        ref = oracle.gemv_bf16_f64(wb, np_ops["x"])
        ok, excess, rel = oracle.close_to_ref(y, ref, RTOL, ATOL)
        assert ok and rel < REF_GATE, (N, K, excess, rel)


def test_contract_checks_on_device_buffers(gemv_lib, cuda):
    """-2 for K % 8/16/128 and misaligned pointers on real allocations (gemv_bf16_check.cu:375-376,474-476)."""
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device=cuda)
    p = buf.data_ptr()
    L = gemv_lib._lib
    assert L.paia_gemv_bf16(p, p, p, 4, 12, 0, None) == -2
    assert L.paia_gemv_fp8(p, p, p, p, 4, 24, 0, None) == -2
    assert L.paia_gemv_int4(p, p, p, p, 4, 64, 0, None) == -2
    assert L.paia_gemv_bf16(p + 2, p, p + 4096, 4, 16, 0, None) == -2
    with pytest.raises(RuntimeError):
        gemv_lib.bf16(p, p, p, 4, 12, 0)
    torch.cuda.synchronize()


def test_deterministic_and_split_k_agrees(oracle, gemv_lib, cuda):
    """Same call twice -> identical bits (fixed reduction order); split-K (H=1) and row-parallel (H=0) variants
    of the same (R,U,W) agree within the gate on the tall-K down_proj."""
    for fmt in ("fp8", "int4zp"):
        N, K = 4096, 14336
        ops, np_ops = make(fmt, N, K)
        dev = to_device(ops, cuda)
        vs = variants(gemv_lib, fmt)
        h0 = next(v["id"] for v in vs if (v["R"], v["U"], v["W"], v["H"]) == (2, 2, 4, 0))
        h1 = next(v["id"] for v in vs if (v["R"], v["U"], v["W"], v["H"]) == (2, 2, 4, 1))
        note(f"determinism {fmt}")
        a = bits16(run_gemv(gemv_lib, fmt, dev, h1))
        b = bits16(run_gemv(gemv_lib, fmt, dev, h1))
        c = bits16(run_gemv(gemv_lib, fmt, dev, h0))
        assert np.array_equal(a, b)
        yb = torch.from_numpy(c.view(np.int16)).view(torch.bfloat16)
        check(oracle, fmt, np_ops, yb, f"{fmt} H=0")


def test_graph_capture_replays_match_eager(oracle, gemv_lib, cuda):
    """A HIP graph of GEMVs in all four formats, replayed several times with eager work in between; every replay
    must equal the eager result bit for bit."""
    cases = []
    for fmt, (N, K) in [("bf16", (1000, 3584)), ("fp8", (4097, 4096)), ("int4", (513, 14336)),
                        ("int4zp", (4608, 3584))]:
        ops, np_ops = make(fmt, N, K, bias=fmt != "int4")
        dev = to_device(ops, cuda)
        kind = fmt
        vid = gemv_lib.pick_variant(kind, N, K)
        eager = bits16(run_gemv(gemv_lib, fmt, dev, vid))
        cases.append((fmt, dev, vid, eager, torch.empty(N, dtype=torch.bfloat16, device=cuda)))
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for fmt, dev, vid, _, y in cases:
            run_gemv(gemv_lib, fmt, dev, vid, y=y)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fmt, dev, vid, _, y in cases:
            run_gemv(gemv_lib, fmt, dev, vid, y=y)
    for rep in range(4):
        for *_, y in cases:
            y.fill_(float("nan"))
        junk = torch.randn(1 << 20, device=cuda).sum()          # eager work between replays
        torch.cuda.synchronize()
        note(f"graph replay {rep}")
        g.replay()
        torch.cuda.synchronize()
        for fmt, _, _, eager, y in cases:
            assert np.array_equal(bits16(y), eager), f"replay {rep} {fmt}"
        del junk


def test_torch_ops_refuse_operands_off_the_weight_device(cuda):
    """The torch ops run whenever any argument is on the GPU, so an operand left in host memory must be refused
    before a kernel could dereference its pointer: x, scale, bias or out on the CPU -> RuntimeError, nothing launched."""
    from paia_gemv import ops
    ops.load()
    N, K = 64, 1024
    Wq = torch.zeros(N, K, dtype=torch.uint8, device=cuda)
    scale = torch.ones(N, dtype=torch.float32, device=cuda)
    x = torch.zeros(K, dtype=torch.bfloat16, device=cuda)
    bias = torch.zeros(N, dtype=torch.bfloat16, device=cuda)
    y = ops.gemv_fp8(Wq, scale, x, bias=bias)                     # all on the GPU: runs
    torch.cuda.synchronize()
    assert y.device == Wq.device and y.shape == (N,)
    for what, args, kw in [("x", (Wq, scale, x.cpu()), {}), ("scale", (Wq, scale.cpu(), x), {}),
                           ("bias", (Wq, scale, x), {"bias": bias.cpu()}),
                           ("out", (Wq, scale, x), {"out": torch.empty(N, dtype=torch.bfloat16)})]:
        note(f"host {what}")
        with pytest.raises(RuntimeError, match="device"):
            ops.gemv_fp8(*args, **kw)
    Wb = torch.zeros(N, K, dtype=torch.bfloat16)                  # weights on the host, x on the GPU
    with pytest.raises(RuntimeError):
        ops.gemv_bf16(Wb, x)
    torch.cuda.synchronize()
