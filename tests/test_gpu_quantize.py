"""GPU parity of the on-device quantizers (paia_quantize_*, through the C ABI and the torch ops) with the CPU oracle:
bit-exact codes, scales and zero points (the formats of src/paia_gemv/quant.py:8-31 and quant_host.h:74-106, plus the
asymmetric INT4 format).

The e4m3 rounding probe makes the hardware convert's rounding visible: a row whose amax is 448 has scale exactly 1,
so the row's other values reach the encoder unchanged; the row holds every midpoint between neighbouring e4m3 codes
and the floats just below and above each midpoint. Rounding to the nearest code is monotone, so agreement there
(ties to the even code included) means agreement for every input.
"""
import numpy as np
import pytest
import torch

from gpu_util import note

pytestmark = pytest.mark.gpu


def _dev(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def run_fp8(lib, W, cuda):
    N, K = W.shape
    d = _dev(W, cuda)
    q = torch.empty(N, K, dtype=torch.uint8, device=cuda)
    s = torch.empty(N, dtype=torch.float32, device=cuda)
    lib.quantize_fp8_rowwise(d.data_ptr(), q.data_ptr(), s.data_ptr(), N, K)
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


def e4m3_probe_rows(oracle):
    t = oracle.e4m3_table()
    fin = np.sort(np.unique(np.abs(t[np.isfinite(t)])))
    mids = ((fin[:-1] + fin[1:]) / 2).astype(np.float32)
    vals = np.concatenate([mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9)), fin,
                           np.float32([0.0, 2.0 ** -12, 2.0 ** -10, 3 * 2.0 ** -11])]).astype(np.float32)
    vals = np.concatenate([vals, -vals])
    K = 1024
    rows = []
    for i in range(0, len(vals), K - 16):
        r = np.zeros(K, np.float32)
        chunk = vals[i:i + K - 16]
        r[:len(chunk)] = chunk
        r[K - 1] = 448.0                                   # amax 448 -> scale exactly 1
        rows.append(r)
    return np.stack(rows)


def test_quantize_fp8_every_rounding_case_bitexact(oracle, gemv_lib, cuda):
    W = e4m3_probe_rows(oracle)
    note(f"quantize fp8 probe {W.shape}")
    q, s = run_fp8(gemv_lib, W, cuda)
    q0, s0 = oracle.quantize_fp8_rowwise(W)
    assert np.all(s == 1.0) and np.array_equal(s, s0)
    bad = np.nonzero(q != q0)
    assert bad[0].size == 0, f"{bad[0].size} codes differ, e.g. value {W[bad][:4]} -> {q[bad][:4]} vs {q0[bad][:4]}"


@pytest.mark.parametrize("N,K", [(1, 16), (37, 1040), (512, 4096), (96, 18944)])
def test_quantize_fp8_seeded_bitexact(oracle, gemv_lib, cuda, N, K):
    rng = np.random.default_rng(N + K)
    W = (rng.standard_normal((N, K)) * rng.uniform(1e-4, 10.0, (N, 1))).astype(np.float32)
    W[0, :] = 0.0                                          # zero row -> scale 1
    if N > 2:
        W[1, 3] = -0.0
        W[2, :] = np.float32(1e-30)                        # tiny row: scale underflows toward denormals
    note(f"quantize fp8 {N}x{K}")
    q, s = run_fp8(gemv_lib, W, cuda)
    q0, s0 = oracle.quantize_fp8_rowwise(W)
    assert np.array_equal(s.view(np.uint32), s0.view(np.uint32)) and np.array_equal(q, q0)


def test_quantize_int4_bitexact_with_ties_and_specials(oracle, gemv_lib, cuda):
    rng = np.random.default_rng(5)
    N, K = 64, 3584
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    W[0, :128] = 0.0                                       # zero group -> fp16 1.0
    W[1, 128:256] = np.float32(1e-9)                       # amax/7 underflows fp16 -> stored 0, quantised with 1
    ties = (np.arange(128) % 15 - 7 + 0.5).astype(np.float32)
    ties[0] = 7.0                                          # amax 7 -> scale exactly 1: every w/s is a .5 tie
    W[2, 256:384] = ties
    G = K // 128
    d = _dev(W, cuda)
    p = torch.empty(N, K // 2, dtype=torch.uint8, device=cuda)
    s = torch.empty(N, G, dtype=torch.float16, device=cuda)
    note(f"quantize int4 {N}x{K}")
    gemv_lib.quantize_int4_g128(d.data_ptr(), p.data_ptr(), s.data_ptr(), N, K)
    torch.cuda.synchronize()
    p0, s0 = oracle.quantize_int4_g128(W)
    assert np.array_equal(s.cpu().view(torch.int16).numpy().view(np.uint16), s0)
    assert np.array_equal(p.cpu().numpy(), p0)


def test_quantize_int4_zp_bitexact(oracle, gemv_lib, cuda):
    rng = np.random.default_rng(6)
    for N, K in [(33, 384), (128, 4096), (16, 18944)]:    # G = 3 (odd), 32, 148
        G = K // 128
        W = (rng.standard_normal((N, K)) * 0.02 + rng.uniform(-0.01, 0.01, (N, 1))).astype(np.float32)
        W[0, :128] = 0.0
        d = _dev(W, cuda)
        p = torch.empty(N, K // 2, dtype=torch.uint8, device=cuda)
        s = torch.empty(N, G, dtype=torch.bfloat16, device=cuda)
        z = torch.full((N, (G + 1) // 2), 0xAB, dtype=torch.uint8, device=cuda)
        note(f"quantize int4 zp {N}x{K}")
        gemv_lib.quantize_int4_zp_g128(d.data_ptr(), p.data_ptr(), s.data_ptr(), z.data_ptr(), N, K)
        torch.cuda.synchronize()
        p0, s0, z0 = oracle.quantize_int4_zp_g128(W)
        assert np.array_equal(p.cpu().numpy(), p0) and np.array_equal(z.cpu().numpy(), z0)
        assert np.array_equal(s.cpu().view(torch.int16).numpy().view(np.uint16), s0)


def test_quant_api_on_device_matches_definition(cuda):
    """paia_gemv.quant on a GPU tensor (the HIP kernels through the torch ops) == the torch definition on the CPU."""
    from paia_gemv import quant
    g = torch.Generator().manual_seed(7)
    W = 0.02 * torch.randn(300, 4096, generator=g)
    note("quant api fp8/int4/int4zp")
    for fn in (quant.quantize_fp8_rowwise, quant.quantize_int4_g128, quant.quantize_int4_zp_g128):
        cpu = fn(W)
        dev = fn(W.to(cuda))
        for a, b in zip(cpu, dev):
            assert a.dtype == b.dtype and torch.equal(a.view(torch.uint8) if a.element_size() == 1 else a,
                                                      (b.view(torch.uint8) if b.element_size() == 1 else b).cpu())
