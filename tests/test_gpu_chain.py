"""the Llama-3.1-8B decode-step linear chain as one HIP graph, through the C ABI.

32 layers x (qkv 6144x4096, o 4096x4096, gate_up 28672x4096, down 4096x14336) in INT4 (asymmetric g128) and in FP8,
then the bf16 lm_head 128256x4096: 129 launches, each layer on its own buffers (paia_bench.chain.build_chain, the
graph bench.py times). The graph is replayed several times with eager work and synchronisations between replays;
every replay must reproduce the eager pass's 129 outputs bit for bit, and sampled rows of every layer's output and
of the lm_head must match the fp64 oracle on that layer's own operands (the reference harness gates each cell before
timing it, paia-bench/bench/run.py:236-240).
"""
import numpy as np
import pytest
import torch

from gpu_util import bits16, note, oracle_ref
from paia_bench.chain import build_chain, sample_rows
from paia_bench.inputs import as_numpy
from paia_bench.timing import capture

pytestmark = pytest.mark.gpu

RTOL = ATOL = 1e-2
REF_GATE = 2e-2


@pytest.mark.parametrize("fmt", ["int4zp", "fp8"])
def test_decode_chain_graph_every_layer(oracle, gemv_lib, cuda, fmt):
    note(f"chain {fmt}: build 32 layers + lm_head")
    launches, total, checks = build_chain(gemv_lib, fmt, device=cuda)
    try:
        assert len(launches) == 32 * 4 + 1
        assert all(v["ok"] for v in checks.values()), checks

        def step():
            for case, i in launches:
                case.call(i)

        note(f"chain {fmt}: eager pass")
        step()
        torch.cuda.synchronize()
        eager = [bits16(case.copies[i]["y"]) for case, i in launches]
        note(f"chain {fmt}: capture")
        g = capture(step)
        for rep in range(3):
            for case, i in launches:
                case.copies[i]["y"].fill_(float("nan"))
            junk = torch.randn(1 << 20, device=cuda).sum()       # eager work between replays
            torch.cuda.synchronize()
            note(f"chain {fmt}: replay {rep}")
            g.replay()
            torch.cuda.synchronize()
            for (case, i), want in zip(launches, eager):
                assert np.array_equal(bits16(case.copies[i]["y"]), want), f"replay {rep}: {case.name} layer {i}"
            del junk
        del g
        # every layer's output (and the head) on sampled rows against the fp64 oracle on its own operands
        worst = 0.0
        for (case, i), yb in zip(launches, eager):
            rows = sample_rows(case.N, 32)
            np_ops = as_numpy(case.copy_rows(i, rows))
            ref = oracle_ref(oracle, case.fmt, np_ops)
            ok, excess, rel = oracle.close_to_ref(yb[rows].copy(), ref, RTOL, ATOL)
            assert ok and rel < REF_GATE, f"{case.name} layer {i}: excess {excess:.3e} rel {rel:.3e}"
            worst = max(worst, rel)
        print(f"chain {fmt}: {len(launches)} outputs match the oracle (worst rel {worst:.2e}), {total / 1e9:.2f} GB")
    finally:
        for case in {c for c, _ in launches}:
            case.free()
        torch.cuda.empty_cache()
