"""The measurement phases' cell sets (no GPU): the reference harness's frozen sets (paia-bench/bench/run.py:72-111,
src/patches/integration_quant.patch:9-60) over paia-bench/configs/shapes.yaml's shapes, and the summary table."""
from paia_bench.phases import MODES, cells, summary
from paia_gemv.shapes import BATCH_M, MODELS, SYNTHETIC


def test_frozen_shape_set_matches_the_reference_config():
    assert [len(Ns) for _, Ns in SYNTHETIC.values()] == [14, 12]           # shapes.yaml:53-60
    assert SYNTHETIC["K4096"][1][0] == 32 and SYNTHETIC["K4096"][1][-1] == 131072
    assert all(len(m) == 10 for m in MODELS.values()) and BATCH_M == [1, 2, 4, 8, 16]


def test_phase_cell_counts_and_modes():
    n_shapes = 14 + 12 + 20
    s1 = cells("s1")
    assert len(s1) == 3 * n_shapes and {c["timing_mode"] for c in s1} == set(MODES)
    assert len(cells("s3")) == 3 * n_shapes                                # every frozen K is a multiple of 16
    s4 = cells("s4")
    assert len(s4) == 5 * n_shapes                                         # fused x 3 modes + naive + unfused
    assert {c["timing_mode"] for c in s4 if c["family"] != "fused"} == {"graph"}
    e2 = cells("e2")
    assert len(e2) == 3 * n_shapes + 20 * 4 and all(c["timing_mode"] == "graph" for c in e2 if c["M"] > 1)
    sb = cells("sb")
    assert len(sb) == 2 * 20 * 5 and {c["M"] for c in sb} == set(BATCH_M)


def test_summary_table():
    recs = [{"phase": "s3", "impl": "paia_gemv_fp8", "model": "llama31_8b", "layer_name": "o_proj", "M": 1,
             "N": 4096, "K": 4096, "timing_mode": m, "median_us": t, "pct_of_8TBps": 40.0}
            for m, t in (("isolated", 9.5), ("eager", 5.1), ("graph", 4.8))]
    text = summary(recs)
    assert "| llama31_8b:o_proj | 1 | 4096x4096 | 9.50 (40.0%) | 5.10 (40.0%) | 4.80 (40.0%) |" in text
