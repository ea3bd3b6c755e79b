"""paia_gemv_int4_unfused_noalloc: the unfused INT4 control without a caller workspace, through the C ABI.

The entry point has no counterpart in the reference; it serves callers that cannot allocate. Its output must equal
paia_gemv_int4_unfused's (the same kernels and BF16 variant, slice by slice over the library's static device scratch)
bit for bit, on consecutive calls whose second is smaller than the first (the scratch then still holds the first
call's rows), including calls that need several slices; and the bf16-weight reference gate of the unfused control
(src/tests/gemv_bf16_check.cu:350-352) holds.
"""
import numpy as np
import pytest
import torch

from gpu_util import bits16, make, nan_filled, note, run_gemv
from paia_bench.inputs import to_device

RTOL = ATOL = 1e-2
REF_GATE = 2e-2
MAX_K = 2097152        # 8 bf16 rows of K values fill the 32 MiB scratch


def test_noalloc_rejects_k_beyond_the_scratch_without_launching(gemv_lib):
    """Host checks only (no GPU needed): K too large for 8 rows of scratch, and the usual contract, return -2."""
    L = gemv_lib._lib
    A = 1 << 20
    assert L.paia_gemv_int4_unfused_noalloc(A, A, A, A, 4, MAX_K + 128, None) == -2
    assert L.paia_gemv_int4_unfused_noalloc(A, A, A, A, 4, 64, None) == -2          # K % 128
    assert L.paia_gemv_int4_unfused_noalloc(A, A, A, A + 2, 4, 128, None) == -2     # y not 16-byte aligned
    assert L.paia_gemv_int4_unfused_noalloc(A, A, A, A, 0, 128, None) == -2         # N <= 0


@pytest.mark.gpu
def test_noalloc_equals_the_unfused_entry_point(oracle, gemv_lib, cuda):
    # 9000x4096: three slices of up to 4096 rows; then a smaller call (one slice) over the stale scratch; then
    # 2500x14336: slices of 1168 rows; 700x65536: slices of 256 rows, the last one ragged, each slice's BF16 GEMV on
    # the x-from-global kernel (K beyond x staging); then a small call again
    for N, K in [(9000, 4096), (1000, 3584), (2500, 14336), (700, 65536), (8, 4096)]:
        ops, np_ops = make("int4", N, K)
        dev = to_device(ops, cuda)
        note(f"noalloc unfused reference call N={N} K={K}")
        scratch = torch.empty(N * K, dtype=torch.bfloat16, device=cuda)
        want = bits16(run_gemv(gemv_lib, "int4", dev, 0, mode="unfused", scratch=scratch))
        del scratch
        note(f"noalloc call N={N} K={K}")
        y = nan_filled(N, cuda)
        gemv_lib.int4_unfused_noalloc(dev["Wq"].data_ptr(), dev["scales"].data_ptr(), dev["x"].data_ptr(),
                                      y.data_ptr(), N, K)
        torch.cuda.synchronize()
        got = bits16(y)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, f"{N}x{K}: {bad.size} rows differ from paia_gemv_int4_unfused, first {bad[:5]}"
        wb = oracle.dequant_int4_bf16(np_ops["Wq"], np_ops["scales"])
        ok, excess, rel = oracle.close_to_ref(got, oracle.gemv_bf16_f64(wb, np_ops["x"]), RTOL, ATOL)
        assert ok and rel < REF_GATE, (N, K, excess, rel)
