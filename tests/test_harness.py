"""Benchmark-harness logic without a GPU: the CPU reference the harness gates on, the rocprofv3 summaries, the tuned
per-shape table and bench.py's one-GPU contract."""
import json
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from paia_bench import pmc, rocprof_summary
from paia_bench.cases import GemvCase
from paia_bench.inputs import as_numpy, make_operands

ROOT = Path(__file__).resolve().parents[1]


class _NoLib:
    def pick_variant(self, kind, N, K):
        return 0


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int4", "int4zp"])
def test_harness_reference_matches_oracle(oracle, fmt):
    """GemvCase.reference (torch dequant + fp32 matmul, the reference harness's method) agrees with the fp64 oracle
    to fp32 accuracy, on all rows and on a row subset, with and without bias."""
    for N, K, bias in [(37, 256, False), (64, 3584, fmt != "int4")]:
        c = GemvCase(_NoLib(), fmt, N, K, bias=bias)
        c.ops0 = make_operands(fmt, N, K, bias=bias)
        a = as_numpy(c.ops0)
        b = a.get("bias")
        ref64 = {"bf16": lambda: oracle.gemv_bf16_f64(a["W"], a["x"], b),
                 "fp8": lambda: oracle.gemv_fp8_f64(a["Wq"], a["scale"], a["x"], b),
                 "int4": lambda: oracle.gemv_int4_f64(a["Wq"], a["scales"], a["x"]),
                 "int4zp": lambda: oracle.gemv_int4_zp_f64(a["Wq"], a["scales"], a["zeros"], a["x"], b)}[fmt]()
        got = c.reference().numpy().astype(np.float64)
        assert np.allclose(got, ref64, rtol=1e-5, atol=1e-5 * np.abs(ref64).max())
        rows = [0, N // 2, N - 1]
        # (BLAS blocking differs with the row count: equal to fp32 rounding, not bit for bit)
        assert np.allclose(c.reference(rows).numpy(), c.reference().numpy()[rows], rtol=1e-6, atol=1e-6)


def _counter_csv(path, rows):
    cols = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    with open(path, "w") as f:
        f.write(",".join(f'"{c}"' for c in cols) + "\n")
        for i, (k, c, v) in enumerate(rows):
            f.write(f'{i},"{k}","{c}",{v}\n')


def test_pmc_summary_calibrates_counters(tmp_path):
    """FETCH_SIZE/WRITE_SIZE (KiB per dispatch) are scaled by what they read for the calibration kernels: a counter
    that reads half the bytes of the known-size read probe is doubled for the GEMV too."""
    cal_kib = pmc.CAL_BYTES / 1024
    k = "void paia::gemv_kernel<1, 2, 2, 4, 2, false>(paia::GemvParams)"
    fetch, write = tmp_path / "f.csv", tmp_path / "w.csv"
    _counter_csv(fetch, [("read_probe_kernel<1>", "FETCH_SIZE", cal_kib / 2), ("copy_probe_kernel", "FETCH_SIZE",
                                                                              cal_kib / 2),
                         (k, "FETCH_SIZE", 57863.0), (k, "FETCH_SIZE", 57860.0), (k, "FETCH_SIZE", 57870.0)])
    _counter_csv(write, [("read_probe_kernel<1>", "WRITE_SIZE", 0.0), ("copy_probe_kernel", "WRITE_SIZE", cal_kib),
                         (k, "WRITE_SIZE", 224.0)])
    out = tmp_path / "t.json"
    pmc.main(["summarize", "--fetch", str(fetch), "--write", str(write), "--out", str(out), "--case", "c1",
              "--fmt", "fp8", "--shape", "28672x4096"])
    d = json.loads(out.read_text())
    assert d["calibration"]["fetch_per_byte_read_probe"] == 0.5
    e = d["cases"]["c1"]
    assert e["fetch_bytes"] == round(57863.0 * 1024 * 2) and e["write_bytes"] == 224 * 1024
    assert e["algorithmic_bytes"] == 117620736 and e["kernel"] == "paia::gemv_kernel<1, 2, 2, 4, 2, false>"


def test_rocprof_trace_summary_groups_by_grid(tmp_path):
    t = tmp_path / "trace.csv"
    cols = ["Kernel_Name", "Grid_Size_X", "Workgroup_Size_X", "Start_Timestamp", "End_Timestamp", "VGPR_Count",
            "SGPR_Count", "LDS_Block_Size", "Scratch_Size"]
    k = "void paia::gemv_kernel<1, 2, 2, 4, 2, false>(paia::GemvParams)"
    rows = [(k, 256 * 1024, 256, 0, 1000), (k, 256 * 1024, 256, 0, 3000), (k, 512 * 1024, 512, 0, 5000),
            ("other", 64, 64, 0, 9)]
    with open(t, "w") as f:
        f.write(",".join(cols) + "\n")
        for r in rows:
            f.write(f'"{r[0]}",{r[1]},{r[2]},{r[3]},{r[4]},40,64,0,0\n')
    s = rocprof_summary.summarize(str(t), "gemv_kernel")
    assert [(r["blocks"], r["threads"], r["calls"], r["avg_ns"]) for r in s] == [(1024, 512, 1, 5000.0), (1024, 256, 2, 2000.0)]
    assert "paia::gemv_kernel<1, 2, 2, 4, 2, false>" in rocprof_summary.to_markdown(s)


def test_tuned_table_drives_pick_variant(gemv_lib):
    """Every entry of the frozen MI355X table is what paia_gemv_pick_variant returns for that shape."""
    tuned = json.loads((ROOT / "paia-project_amd" / "tuned" / "mi355x.json").read_text())
    fams = {"shapes": ("bf16", gemv_lib.variants), "fp8_shapes": ("fp8", gemv_lib.variants_fp8),
            "int4_shapes": ("int4", gemv_lib.variants_int4), "int4zp_shapes": ("int4zp", gemv_lib.variants_int4)}
    n = 0
    for sec, (kind, fam) in fams.items():
        for key, e in tuned.get(sec, {}).items():
            N, K = map(int, key.split("x"))
            v = fam[gemv_lib.pick_variant(kind, N, K)]
            assert all(v[k] == e["variant"][k] for k in "RUWH"), (sec, key, v, e["variant"])
            n += 1
    assert n >= 30


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_sweep_merge_writes_the_faster_cell(tmp_path):
    """`paia_bench.sweep --merge A B --write-tuned T`: per cell the faster of the files' best variants, M = 1 cells
    under the format's section, "MxNxK" cells under its batch section, and existing entries of other cells kept."""
    from paia_bench import sweep

    def res(us_m1, us_b, v_b):
        return {"fmt": "fp8", "results": {
            "4096x4096": {"ranked": [{"variant": {"R": 2, "U": 2, "W": 4, "S": 0, "H": 0}, "us": us_m1, "gbps": 1.0}]},
            "5x4096x4096": {"ranked": [{"variant": v_b, "us": us_b, "gbps": 1.0}]},
            "8x1x1": {"ranked": []}}}
    rows = {"P": 0, "U": 2, "W": 8, "S": 1, "X": 5}
    mfma = {"P": 1, "U": 2, "W": 8, "S": 8, "X": 1}
    a, b, t = tmp_path / "a.json", tmp_path / "b.json", tmp_path / "t.json"
    a.write_text(json.dumps(res(5.0, 6.5, rows)))
    b.write_text(json.dumps(res(4.0, 7.7, mfma)))
    t.write_text(json.dumps({"platform": "mi355x", "fp8_shapes": {"1x2": {"variant": {}}}}))
    assert sweep.main(["--fmt", "fp8", "--merge", str(a), str(b), "--write-tuned", str(t)]) == 0
    out = json.loads(t.read_text())
    assert out["fp8_shapes"]["4096x4096"]["us"] == 4.0 and "1x2" in out["fp8_shapes"]
    assert out["fp8_batch_shapes"]["5x4096x4096"]["variant"] == rows
    assert "8x1x1" not in out["fp8_batch_shapes"]


def test_probe_slices_stay_inside_the_buffer():
    """The read-floor probe rotates reads of S bytes over slices of its buffer: every slice must lie wholly inside it,
    for every GEMV of the benchmark (the 1.09 GB lm_heads leave room for one slice only), and a read larger than the
    buffer is refused on the host."""
    import bench
    from paia_bench.probe import slice_plan
    from paia_gemv.shapes import gemv_bytes
    sizes = [gemv_bytes(f, N, K, b)["total"] for _, f, _, _, N, K, b in bench.PER_GEMV]
    assert max(sizes) > bench.B0_BYTES // 2                      # the case that needs a single slice
    for S in sizes + [1, 255, 256, 257, bench.B0_BYTES - 1, bench.B0_BYTES]:
        stride, n = slice_plan(bench.B0_BYTES, S)
        assert stride >= S and stride % 256 == 0 and n >= 1
        assert (n - 1) * stride + S <= bench.B0_BYTES, (S, stride, n)
    for S in (0, bench.B0_BYTES + 1):
        with pytest.raises(ValueError):
            slice_plan(bench.B0_BYTES, S)


def test_every_probe_shape_is_instantiated():
    """Each GEMV-path probe shape the benchmark sweeps is one the probe library launches: the entry point rejects an
    unknown (U, W) with -1 before looking at its buffers, so null buffers tell the two apart without a GPU (-2)."""
    from paia_bench.probe import PROBE_CONFIGS, SIZED_CONFIGS, load_probe
    P = load_probe()
    for cfg in set(PROBE_CONFIGS) | set(SIZED_CONFIGS):
        if cfg[0] == "st":
            assert P.paia_probe_stream(None, 1 << 20, None, cfg[1], cfg[2], 256 * cfg[3], None) == -2, cfg
        elif cfg[0] == "lw":
            assert P.paia_probe_stream_lead(None, 1 << 20, None, cfg[1], 256 * cfg[2], None) == -2, cfg
    assert P.paia_probe_stream(None, 1 << 20, None, 16, 16, 256, None) == -1       # spills: not instantiated
    assert P.paia_probe_stream(None, 1 << 20, None, 4, 1, 256, None) == -1
    assert P.paia_probe_stream_lead(None, 1 << 20, None, 4, 256, None) == -1


def test_probe_output_setting_is_checked():
    """The I/O-floor output of the read probes: refused without a buffer, odd-aligned or >= 2^31 values; nout = 0
    (the default) turns the writes off. No GPU work."""
    from paia_bench.probe import load_probe
    P = load_probe()
    assert P.paia_probe_set_output(None, 4096) == -2
    assert P.paia_probe_set_output(1, 4096) == -2                  # not 2-byte aligned
    assert P.paia_probe_set_output(2, 1 << 31) == -2
    assert P.paia_probe_set_output(2, 4096) == 0
    assert P.paia_probe_set_output(None, 0) == 0


def test_staged_probe_argument_checks():
    """The staged-x read probe refuses null or unaligned buffers and x sizes outside 1024..65536 bytes or not a
    multiple of 16, before any GPU work."""
    from paia_bench.probe import load_probe
    P = load_probe()
    assert P.paia_probe_read_staged(None, 1 << 20, 16, 256, 16, 8192, None) == -2
    assert P.paia_probe_read_staged(16, 1 << 20, 16, 256, None, 8192, None) == -2
    assert P.paia_probe_read_staged(8, 1 << 20, 16, 256, 16, 8192, None) == -2     # buffer not 16-byte aligned
    assert P.paia_probe_read_staged(16, 1 << 20, 16, 256, 16, 512, None) == -2     # x below 1024 bytes
    assert P.paia_probe_read_staged(16, 1 << 20, 16, 256, 16, 8200, None) == -2    # not a multiple of 16
    assert P.paia_probe_read_staged(16, 1 << 20, 16, 256, 16, 65552, None) == -2   # above 64 KiB
    assert P.paia_probe_read_staged(16, 1 << 20, 16, 0, 16, 8192, None) == -2      # no blocks


@pytest.mark.gpu
def test_traffic_entries_match_their_kernel(gemv_lib):
    """bench.py attaches a committed counter summary to a case only when it was measured on the kernel the case runs
    now, and every committed entry names the kernel the library picks for its case today (a retuned pick needs its
    counters measured again). On the GPU: the kernel a launch runs depends on the device's occupancy figures."""
    import bench
    d = json.loads((Path(bench.__file__).parent / "profiles" / "pmc_traffic.json").read_text())
    shapes = {bench.case_name(f, m, nm, N, K, b): (f, N, K) for _, f, m, nm, N, K, b in bench.PER_GEMV}
    for name, e in d["cases"].items():
        assert bench.load_traffic(name, e["kernel"])["bytes"] == round(e["traffic_bytes"])
        assert bench.load_traffic(name, e["kernel"] + "x") is None
        f, N, K = shapes[name]
        assert e["kernel"] == bench.kernel_name(gemv_lib, f, gemv_lib.pick_variant(f, N, K), N, K), name


def _full_record_fixture():
    """A full bench record of the shape main() builds (every BASELINE GEMV, B0 read floors, both chains, every CPU
    row), with values of the size a real run prints."""
    import bench
    per, floors, cpu_rows = {}, {}, []
    for cfg, f, m, nm, N, K, b in bench.PER_GEMV:
        name = bench.case_name(f, m, nm, N, K, b)
        per[name] = {"config": cfg, "N": N, "K": K, "us": 152.365, "gbps": 7156.3, "pct_of_8TBps": 89.5,
                     "variant": {"id": 63, "R": 2, "U": 8, "W": 8, "S": 1, "H": 1},
                     "kernel": "paia::gemv_kernel<0, 2, 8, 8, 2, true>", "bytes": 1090306048, "R": 32, "copies": 2,
                     "us_allocations": [152.361, 153.087, 153.223, 152.1, 152.9],
                     "samples_per_allocation": [44, 44, 44, 44, 44], "alloc_spread_pct": 0.415, "rel_err": 0.00211,
                     "traffic_over_algorithmic": 1.0045, "pct_of_b0": 96.4, "over_read_floor": 1.037,
                     "over_io_floor": 1.032}
        floors[name] = {"bytes": 1090306048, "us": 147.973, "gbps": 7368.2, "cfg": ["lw", 16, 2], "io_us": 148.661,
                        "io_cfg": ["lw", 16, 2], "nout": N}
        cpu_rows.append({"config": cfg, "gemv": name, "bytes": 1090306048, "us_dequant_matmul": 123456.7,
                         "us_matmul": 23456.7, "gbps_dequant_matmul": 1.555, "gbps_matmul": 4.321})
    roof = {"bound": "hbm", "achieved": 6270.3, "peak": 8000.0, "unit": "GB/s", "frac": 0.7838,
            "traffic": 118144334, "kernel": "paia::gemv_kernel<1, 2, 2, 4, 2, false>",
            "case": "fp8_llama_gate_up_28672x4096", "avg_launch_us": 18.759, "algorithmic_bytes": 117620736,
            "traffic_detail": {"bytes": 118144334, "kernel": "paia::gemv_kernel<1, 2, 2, 4, 2, false>",
                               "fetch_bytes": 117919054, "write_bytes": 225280, "over_algorithmic": 1.0045}}
    chain = {f: {"format": f, "model": "llama31_8b", "bytes_per_step": 8040221184, "gbps": 5473.2,
                 "pct_of_8TBps": 68.4, "us_per_token_step": 1469.21, "us_p5": 1468.1, "us_p95": 1471.9,
                 "replays": 20, "launches": 129, "max_rel_err": 0.0021,
                 "replayed_outputs_checked": [f"x@{i}" for i in range(13)], "replayed_max_rel_err": 0.0021}
             for f in ("int4zp", "fp8")}
    cpu = {"value": 1.624, "unit": "GB/s", "cores": 16, "kind": "port",
           "sample": "23 BASELINE GEMVs once per run (configs[0]-[4]: FP8, INT4-asym, BF16 at the Llama and Qwen "
                     "shapes, lm_heads), seeded copy-0 operands; torch dequant + fp32 matmul, 16 threads, median of "
                     "5 after 2 warm-ups; value = FP8 layer step (configs[1])",
           "cpu": "AMD EPYC 9575F 64-Core Processor", "us_fp8_layer_step": 134567.8,
           "us_fp8_layer_step_matmul_only": 23456.7, "gbps_fp8_layer_step_matmul_only": 9.3,
           "per_config": cpu_rows, "skipped": [], "wall_s": 41.2}
    return {"metric": bench.METRIC, "value": 5305.2, "unit": "GB/s", "n_gpus": 1, "steps": 200, "warmup": 20,
            "ms_per_step": 0.041171, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp8e4m3 weights x bf16 activations, fp32 accumulate",
            "data": "synthetic (seeded N(0,0.02) weights quantised to e4m3fn; N(0,1) bf16 x)",
            "config": {"workload": "FP8 W8A16 GEMV, M=1, Llama-3.1-8B layer: qkv 6144x4096, o 4096x4096, "
                                   "gate_up 28672x4096, down 4096x14336 (BASELINE configs[1])",
                       "layer_copies": 5, "rotation_bytes": 1091927040, "step_bytes": 218385408,
                       "us_per_layer_step": 41.171, "pct_of_8TBps": 66.3, "timed_graph_primed": True},
            "roofline": roof, "roofline_by_dtype": {"bf16": roof, "fp8": roof, "int4zp": roof}, "per_gemv": per,
            "b0": {"gbps": 7389.1, "pct_of_8TBps": 92.4, "bytes": 2146435072, "cfg": ["lw", 16, 2],
                   "read_floor": floors},
            "chain": chain, "cpu_baseline": cpu, "device": "AMD Instinct MI355X", "cus": 256,
            "timed_wall_ms": 8.3}


def test_bench_line_is_compact():
    """The one JSON line the driver parses stays under 4 KB with every field a full run fills (a 21.5 KB line
    arrives truncated and unparsed), carries the contract keys, the dominant kernel's roofline with its
    traffic, one roofline per format, every per-GEMV case and the CPU baseline summary."""
    import bench
    full = _full_record_fixture()
    line = json.dumps(bench.compact_line(full, "out/bench_report.json"))
    assert len(line) < 4096, len(line)
    out = json.loads(line)
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config"):
        assert out[k] == full[k], k
    assert out["roofline"]["traffic"] == 118144334 and out["roofline"]["frac"] == 0.7838
    assert set(out["roofline_by_dtype"]) == {"bf16", "fp8", "int4zp"}
    assert set(out["per_gemv"]) == set(full["per_gemv"]) and len(out["per_gemv"]) == len(bench.PER_GEMV)
    assert out["per_gemv"]["fp8_llama_o_4096x4096"] == [152.365, 89.5, 1.032]
    cpu = out["cpu_baseline"]
    assert cpu["cores"] == 16 and cpu["kind"] == "port" and cpu["gemvs_timed"] == len(bench.PER_GEMV)
    assert out["chain"]["fp8"] == [1469.21, 5473.2, 68.4]
    # a run with the optional legs skipped still forms the line
    bare = dict(full, roofline=None, roofline_by_dtype={}, per_gemv={}, b0=None, chain=None, cpu_baseline=None)
    assert json.loads(json.dumps(bench.compact_line(bare)))["per_gemv"] == {}


def test_pmc_summary_of_every_case_assigns_dispatches_in_order(tmp_path):
    """`summarize --all`: the GEMV dispatches of a counter pass go to the plan's cases in dispatch order, each slice
    checked against its case's kernel; a pass with a dispatch missing, or a slice running another kernel, is refused."""
    cal_kib = pmc.CAL_BYTES / 1024
    ka = "void paia::gemv_kernel<1, 2, 2, 4, 2, false>(paia::GemvParams)"
    kb = "void paia::gemv_kernel43<3, 1, 1, 8, 2, false>(paia::GemvParams)"
    plan = [{"case": "a", "fmt": "fp8", "N": 28672, "K": 4096, "bias": False, "variant": 0,
             "kernel": "paia::gemv_kernel<1, 2, 2, 4, 2, false>", "dispatches": 3},
            {"case": "b", "fmt": "int4zp", "N": 4096, "K": 4096, "bias": False, "variant": 0,
             "kernel": "paia::gemv_kernel43<3, 1, 1, 8, 2, false>", "dispatches": 2}]
    (tmp_path / "plan.json").write_text(json.dumps(plan))
    probes = [("read_probe_kernel<1>", cal_kib / 2), ("copy_probe_kernel", cal_kib / 2)]
    fetch, write = tmp_path / "f.csv", tmp_path / "w.csv"
    _counter_csv(fetch, [(k, "FETCH_SIZE", v) for k, v in probes] +
                 [(ka, "FETCH_SIZE", 57500.0)] * 3 + [(kb, "FETCH_SIZE", 4300.0)] * 2)
    _counter_csv(write, [("read_probe_kernel<1>", "WRITE_SIZE", 0.0), ("copy_probe_kernel", "WRITE_SIZE", cal_kib)] +
                 [(ka, "WRITE_SIZE", 112.0)] * 3 + [(kb, "WRITE_SIZE", 8.0)] * 2)
    out = tmp_path / "t.json"
    args = ["summarize", "--all", "--cases", str(tmp_path / "plan.json"), "--fetch", str(fetch), "--write",
            str(write), "--out", str(out)]
    assert pmc.main(args) == 0
    d = json.loads(out.read_text())["cases"]
    assert d["a"]["fetch_bytes"] == round(57500.0 * 1024 * 2) and d["a"]["dispatches"] == 3
    assert d["b"]["kernel"] == plan[1]["kernel"] and d["b"]["write_bytes"] == 8 * 1024
    plan[1]["kernel"] = "paia::gemv_kernel<3, 1, 1, 8, 2, false>"     # the slice runs another kernel
    (tmp_path / "plan.json").write_text(json.dumps(plan))
    with pytest.raises(SystemExit):
        pmc.main(args)
    plan[1]["dispatches"] = 3                                         # one dispatch more than the pass holds
    plan[1]["kernel"] = "paia::gemv_kernel43<3, 1, 1, 8, 2, false>"
    (tmp_path / "plan.json").write_text(json.dumps(plan))
    with pytest.raises(SystemExit):
        pmc.main(args)
