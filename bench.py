#!/usr/bin/env python3
"""Benchmark of the paia_gemv hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--report PATH] [--no-cpu] [--no-chain] [--no-b0]
                    [--no-per-gemv] [--allocations A]

Workload (the metric's configuration): FP8 W8A16 M=1 GEMVs at the Llama-3.1-8B per-layer shapes
qkv 6144x4096, o 4096x4096, gate_up 28672x4096, down 4096x14336, OCP e4m3fn weights with a per-row fp32 scale, bf16
activations and outputs. One step = the four GEMVs of one decoder layer; steps rotate over L distinct layer copies
whose total (>= 4 x 256 MiB) defeats the Infinity Cache, so every weight byte comes from HBM. The timed region is one
hipGraph replay of K steps (that graph launched once, untimed, beforehand), bracketed by device synchronisation,
with all inputs resident in HBM. Each GEMV uses the library's per-shape variant (paia_gemv_pick_variant, the frozen
MI355X sweep in paia-project_amd/tuned/mi355x.json).

Printed: ONE JSON line, last on stdout and under 4 KB (the driver's contract; `compact_line`), with value = the
aggregate algorithmic GB/s of the FP8 layer step, plus
  roofline          the dominant kernel of the workload (FP8 gate_up): algorithmic bytes / its average launch time
                    (hipEvents on the launch stream, inside this run) vs 8 TB/s; traffic = HBM bytes per launch from the
                    committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary (profiles/pmc_traffic.json), calibrated on
                    kernels of known size. roofline_by_dtype: the same for each format's dominant Llama GEMV
  per_gemv          {case: [us, % of 8 TB/s, GEMV time / I/O floor]} for every GEMV of the BASELINE configs, each
                    shape on its own graph of R back-to-back launches rotating over >= 4 x 256 MiB of copies of that
                    shape alone: configs[0] BF16 o_proj, configs[1] the four FP8 Llama shapes, configs[2] the four INT4
                    (asymmetric g128) Llama shapes, configs[3] the Qwen2.5-7B shapes in all three formats (qkv with
                    its bias) and the bf16 lm_head, configs[4]'s bf16 Llama lm_head; each case on A (default 5)
                    independent allocations, each gated (copy 0 against the CPU reference) before it is timed, the
                    median across them reported
  b0                the streaming-read probe in the same run (the reference's measured-bandwidth denominator "B0"):
                    the best rate of a 2 GiB (less 1 MiB) read; per GEMV byte count it also gives the read floor and
                    the I/O floor (the same reads also writing the GEMV's N bf16 outputs) under the same cold-cache
                    rotation (skipped with --no-b0)
  chain             BASELINE configs[4]: 32 layers x 4 GEMVs + bf16 lm_head as one hipGraph, INT4 (asymmetric g128)
                    and FP8: [us per token-step, GB/s, % of 8 TB/s]; layer 0 gated before capture, layers 0, 1, 31
                    and the head after the replays (skipped with --no-chain)
  cpu_baseline      the reference's CPU path: the paia_gemv.quant torch dequantisation
                    (src/paia_gemv/quant.py semantics) and a torch fp32 matmul (paia-bench/bench/ops/ours_quant.py:
                    69-71) on the host cores, for every GEMV of the BASELINE configs, timed (i) dequant + matmul and
                    (ii) matmul on pre-dequantised weights, median of 5 after 2 warm-ups; value = the FP8 layer
                    step's GB/s under (i)
The full record (per-allocation times, read floors, chain details, every CPU row, counter traffic per case) goes to
--report PATH as indented JSON; stderr carries a few progress lines only.
Copy 0 of every operand set is checked against the CPU fp32 reference (torch dequantisation + matmul, the reference
harness's gate) before anything is timed. The CPU oracle is not used here.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "paia-project_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "µs/GEMV + achieved HBM GB/s (% of 8 TB/s), Llama-3.1-8B shapes, batch 1"
PEAK_GBPS = 8000.0
B0_BYTES = 2 * 2 ** 30 - 2 ** 20   # the B0 read (the GEMV-path probe takes < 2 GiB per launch)

from paia_bench.cases import BASELINE_GEMVS as PER_GEMV, LLAMA_LAYER as LLAMA, case_name, kernel_name  # noqa: E402

# each format's dominant Llama GEMV (roofline_by_dtype): configs[0]'s only shape for BF16, gate_up otherwise
DOMINANT = {"bf16": "bf16_llama_o_4096x4096", "fp8": "fp8_llama_gate_up_28672x4096",
            "int4zp": "int4zp_llama_gate_up_28672x4096"}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def measure_b0(dev, cases, per: dict, log=lambda m: None) -> dict:
    """B0 (the reference's measured streaming-read bandwidth, src/tests/gemv_bf16_check.cu:228-252) in this run: the
    best rate of a 2 GiB (less 1 MiB) read over the probe's launch shapes, then, for each GEMV case (name, bytes, N),
    the read floor for its byte count (reads of that size rotating over the 2 GiB buffer, back to back in one graph)
    and the I/O floor (the same reads that also write the GEMV's N bf16 outputs). Adds pct_of_b0, over_read_floor and
    over_io_floor (GEMV µs / floor µs) to each per_gemv entry."""
    import torch
    from paia_bench.probe import b0_large, b0_sized, load_probe

    P = load_probe()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    buf = torch.empty(B0_BYTES, dtype=torch.uint8, device=dev)
    buf.random_(0, 255)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    gbps, cfg = b0_large(P, buf, sink, cus, log=lambda m: None)
    y = torch.empty(max(n for _, _, n in cases), dtype=torch.bfloat16, device=dev)
    sized = {}
    for name, nbytes, nout in cases:
        r = b0_sized(P, buf, sink, cus, nbytes, y=y, nout=nout)
        sized[name] = {"bytes": r["bytes"], "us": round(r["us"], 3), "gbps": round(r["gbps"], 1), "cfg": r["cfg"],
                       "io_us": round(r["io_us"], 3), "io_cfg": r["io_cfg"], "nout": nout}
        e = per[name]
        e["pct_of_b0"] = round(100 * e["gbps"] / gbps, 1)
        e["over_read_floor"] = round(e["us"] / r["us"], 3)
        e["over_io_floor"] = round(e["us"] / r["io_us"], 3)
    del buf, y
    torch.cuda.empty_cache()
    return {"gbps": round(gbps, 1), "pct_of_8TBps": round(100 * gbps / PEAK_GBPS, 1), "bytes": B0_BYTES,
            "cfg": cfg, "read_floor": sized}


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it, with its family / model / stepping numbers (a virtualised host may
    report only the vendor line as the model name) and the machine's logical CPU count."""
    import platform
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k in ("model name", "cpu family", "model", "stepping") and k not in info:
                info[k] = v.strip()
    except OSError:
        pass
    name = info.get("model name") or platform.processor() or "unknown CPU"
    ids = ", ".join(f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info)
    return f"{name} ({ids}{', ' if ids else ''}{os.cpu_count()} logical CPUs)"


def cpu_baseline(budget_s: float = 90.0) -> dict:
    """The reference's CPU path for every GEMV of the BASELINE configs (PER_GEMV, in its
    order): the seeded operands of the GPU run (paia_bench.inputs.make_operands, CPU generator seeded 1000 + N + K),
    dequantised with paia_gemv.quant's torch definitions (the formulas of src/paia_gemv/quant.py:16-17,34-38; (q - z) * s
    for the asymmetric INT4 format; bf16 -> fp32 for BF16) and multiplied x.float() @ Wdeq.t() in fp32
    (paia-bench/bench/ops/ours_quant.py:69-71, cublas_bf16.py:36), + bias, rounded to bf16. Timed per GEMV as
    (i) dequant + matmul and (ii) matmul on pre-dequantised weights, median of 5 runs after 2 warm-ups
    (time.perf_counter_ns), on all the host cores this process may use (capped by OMP_NUM_THREADS, the box's CPU
    share). GEMVs left when `budget_s` of wall time has passed are not timed (named in `skipped`).
    `value`: the FP8 Llama layer step (configs[1], the metric's workload) under (i), in algorithmic GB/s."""
    import torch
    from paia_bench.inputs import make_operands
    from paia_gemv import quant
    from paia_gemv.shapes import gemv_bytes

    threads = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        threads = min(threads, int(omp))          # the box's CPU share for this job
    torch.set_num_threads(threads)

    def med(fn, reps=5, warm=2):
        for _ in range(warm):
            fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter_ns()
            fn()
            ts.append(time.perf_counter_ns() - t0)
        return statistics.median(ts) / 1e3

    rows, skipped = [], []
    t_start = time.perf_counter()
    for cfg, fmt, model, nm, N, K, bias in PER_GEMV:
        name = case_name(fmt, model, nm, N, K, bias)
        if time.perf_counter() - t_start > budget_s:
            skipped.append(name)
            continue
        o = make_operands(fmt, N, K, bias=bias)
        x = o["x"].float()[None, :]
        b = o["bias"].float() if bias else None

        def deq():
            if fmt == "fp8":
                return quant.dequant_fp8(o["Wq"], o["scale"])
            if fmt == "int4zp":
                return quant.dequant_int4_zp(o["Wq"], o["scales"], o["zeros"])
            return o["W"].float()

        def epi(y):
            return (y if b is None else y + b).to(torch.bfloat16)

        def full():
            return epi(x @ deq().t())

        Wd = deq()

        def mm():
            return epi(x @ Wd.t())

        us_full, us_mm = med(full), med(mm)
        nbytes = gemv_bytes(fmt, N, K, bias)["total"]
        rows.append({"config": cfg, "gemv": name, "bytes": nbytes,
                     "us_dequant_matmul": round(us_full, 1), "us_matmul": round(us_mm, 1),
                     "gbps_dequant_matmul": round(nbytes / us_full / 1e3, 3),
                     "gbps_matmul": round(nbytes / us_mm / 1e3, 3)})
        del Wd, o
    step = [r for r in rows if r["config"] == "configs[1]"]
    step_us = sum(r["us_dequant_matmul"] for r in step)
    step_mm = sum(r["us_matmul"] for r in step)
    step_bytes = sum(r["bytes"] for r in step)
    return {"value": round(step_bytes / step_us / 1e3, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{len(rows)} BASELINE GEMVs once per run (configs[0]-[4]: FP8, INT4-asym, BF16 at the Llama and "
                      f"Qwen shapes, lm_heads), seeded copy-0 operands; torch dequant + fp32 matmul, {threads} "
                      f"threads, median of 5 after 2 warm-ups; value = FP8 layer step (configs[1])",
            "cpu": cpu_model(), "us_fp8_layer_step": round(step_us, 1),
            "us_fp8_layer_step_matmul_only": round(step_mm, 1),
            "gbps_fp8_layer_step_matmul_only": round(step_bytes / step_mm / 1e3, 3) if step_mm else None,
            "per_config": rows, "skipped": skipped, "wall_s": round(time.perf_counter() - t_start, 1)}


def load_traffic(case_name: str, kernel: str):
    """HBM bytes per launch of this GEMV case from the committed rocprofv3 PMC summary (profiles/pmc_traffic.json,
    written by `python -m paia_bench.pmc summarize`), or None if that case was not profiled with this kernel."""
    f = ROOT / "profiles" / "pmc_traffic.json"
    if not f.exists():
        return None
    try:
        d = json.loads(f.read_text())
        e = d.get("cases", {}).get(case_name)
        return None if e is None or e.get("kernel") != kernel else {"bytes": round(e["traffic_bytes"]), "kernel": e.get("kernel"),
                                       "fetch_bytes": round(e["fetch_bytes"]), "write_bytes": round(e["write_bytes"]),
                                       "over_algorithmic": e.get("traffic_over_algorithmic")}
    except (OSError, ValueError, KeyError):
        return None


def roofline_entry(lib, name, e):
    traffic = load_traffic(name, e["kernel"])
    return {"bound": "hbm", "achieved": e["gbps"], "peak": PEAK_GBPS, "unit": "GB/s",
            "frac": round(e["gbps"] / PEAK_GBPS, 4), "traffic": traffic["bytes"] if traffic else None,
            "kernel": e["kernel"], "case": name, "avg_launch_us": e["us"], "algorithmic_bytes": e["bytes"],
            "traffic_detail": traffic}


def measure_per_gemv(lib, dev, allocations: int | None = None) -> dict:
    """Every GEMV of PER_GEMV on its own rotation (>= 4 x 256 MiB of copies of that shape), on `allocations`
    independent allocations (default 5, as the reference), each built, gated (copy 0, sampled rows), timed and
    freed in turn, with R sized on the first and kept; the reported time is the median across them (the reference
    harness's cell protocol, paia-bench/configs/shapes.yaml:72-80, paia-bench/bench/run.py:200-270: fresh
    allocations of one op differ by physical placement)."""
    import torch
    from paia_bench.cases import GemvCase
    from paia_bench.chain import sample_rows
    from paia_bench.timing import ALLOCATIONS_PER_CELL, CELL_SAMPLE_TARGET_MS, plan_rotation, time_per_call_us

    per = {}
    for cfg, fmt, model, nm, N, K, bias in PER_GEMV:
        name = case_name(fmt, model, nm, N, K, bias)
        us_a, n_a, worst, R = [], [], 0.0, None
        k = max(1, ALLOCATIONS_PER_CELL if allocations is None else allocations)
        for _ in range(k):
            c = GemvCase(lib, fmt, N, K, bias=bias, name=name)
            n_rot = plan_rotation(c.footprint())["n_copies"]
            c.build(n_rot, dev, host_copy0=False)
            c.call(0)
            chk = c.check_copy(0, sample_rows(N, 256))
            if not chk["ok"]:
                raise RuntimeError(f"{name} failed the correctness gate: {chk}")
            worst = max(worst, chk["rel_err"])
            t = time_per_call_us(c.call, n_rot, sample_target_ms=CELL_SAMPLE_TARGET_MS / k, R=R)
            R = t["R"]
            us_a.append(t["us"])
            n_a.append(t["us_n"])
            c.free()
            torch.cuda.empty_cache()
        us = statistics.median(us_a)
        gbps = c.bytes()["total"] / (us * 1e-6) / 1e9
        fam = {"bf16": lib.variants, "fp8": lib.variants_fp8}.get(fmt, lib.variants_int4)
        per[name] = {"config": cfg, "N": N, "K": K, "us": round(us, 3), "gbps": round(gbps, 1),
                     "pct_of_8TBps": round(100 * gbps / PEAK_GBPS, 1), "variant": fam[c.variant],
                     "kernel": kernel_name(lib, fmt, c.variant, N, K), "bytes": c.bytes()["total"], "R": t["R"],
                     "copies": n_rot, "us_allocations": [round(u, 3) for u in us_a], "samples_per_allocation": n_a,
                     "alloc_spread_pct": round(100 * (max(us_a) - min(us_a)) / us, 3), "rel_err": round(worst, 5)}
        tr = load_traffic(name, per[name]["kernel"])
        per[name]["traffic_over_algorithmic"] = tr["over_algorithmic"] if tr else None
    log(f"per-GEMV: {len(per)} cases timed")
    return per


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--report", type=str, default=None, help="also write a detailed JSON report here")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-b0", action="store_true", help="skip the streaming-read probe (B0) leg")
    ap.add_argument("--no-chain", action="store_true", help="skip the decode-chain (configs[4]) measurement")
    ap.add_argument("--no-per-gemv", action="store_true", help="skip the per-GEMV figures (and b0, roofline)")
    ap.add_argument("--allocations", type=int, default=None,
                    help="independent operand allocations per per-GEMV case (default 5); the median across them is "
                         "reported")
    a = ap.parse_args(argv)
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {a.gpus}). The M=1 GEMV shards along N "
              "with no collective (each GPU streams its N/g rows with the full x), so the one-GPU figure on one "
              "GPU's share is what this benchmark reports. Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch
    from paia_bench.cases import GemvCase
    from paia_bench.timing import LLC_BYTES, capture
    from paia_gemv import load_lib

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (MI355X)", file=sys.stderr)
        return 3
    lib = load_lib()
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(0)
    log(f"device {props.name} CUs {props.multi_processor_count} lib {lib.path}")

    cases = [GemvCase(lib, "fp8", N, K, name=case_name("fp8", "llama", nm, N, K, False)) for nm, N, K in LLAMA]
    layer_bytes = sum(c.footprint() for c in cases)
    L = max(2, math.ceil(4 * LLC_BYTES / layer_bytes))
    for c in cases:
        c.build(L, dev)
    worst = 0.0
    for c in cases:
        chk = c.check()
        worst = max(worst, chk["rel_err"])
        if not chk["ok"]:
            print(json.dumps({"error": f"{c.name} failed the correctness gate", **chk}))
            return 1

    step_bytes = sum(c.bytes()["total"] for c in cases)

    def steps_fn(n):
        def run():
            for s in range(n):
                for c in cases:
                    c.call(s % L)
        return run

    # warmup replays, then the timed replay of exactly K steps, bracketed by device synchronisation; the events are
    # recorded on the stream the GEMVs launch on (torch's current stream, which the ctypes calls use)
    g_warm = capture(steps_fn(max(1, a.warmup)), warm=1)
    g_timed = capture(steps_fn(a.steps), warm=0)
    g_warm.replay()
    torch.cuda.synchronize()
    # The first launch of an executable graph does one-time per-node setup on MI355X (measured: the first replay of
    # this 800-launch graph ran 41.8-42.1 us/step, every later one 40.5-40.7, with or without hipGraphUpload). That
    # setup is not per-step work, so the timed graph is launched once, untimed, before the timed replay: the run
    # does W + K untimed steps in all (reported as config.timed_graph_primed).
    g_timed.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    g_timed.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = gpu_ms / a.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"{L} layer copies ({L * layer_bytes / 2**30:.2f} GiB), copy 0 gated (worst rel err {worst:.2e}); timed "
        f"{a.steps} steps: {gpu_ms:.3f} ms (wall {wall_ms:.3f} ms), {ms_per_step * 1e3:.2f} us/step, {value:.0f} GB/s")
    del g_warm, g_timed
    for c in cases:
        c.free()
    torch.cuda.empty_cache()

    per, roof, by_dtype, b0 = {}, None, {}, None
    if not a.no_per_gemv:
        per = measure_per_gemv(lib, dev, a.allocations)
        dom = DOMINANT["fp8"]
        roof = roofline_entry(lib, dom, per[dom])
        by_dtype = {f: roofline_entry(lib, n, per[n]) for f, n in DOMINANT.items()}
        if not a.no_b0:
            b0 = measure_b0(dev, [(n, e["bytes"], e["N"]) for n, e in per.items()], per)
            log(f"b0 {b0['gbps']:.0f} GB/s ({b0['pct_of_8TBps']:.1f}% of 8 TB/s)")

    chain = None
    if not a.no_chain:
        from paia_bench.chain import run_chain
        chain = {f: run_chain(lib, f, log=log) for f in ("int4zp", "fp8")}

    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline()
        log(f"cpu {cpu['value']:.2f} GB/s on {cpu['cores']} threads, {len(cpu['per_config'])} GEMVs in "
            f"{cpu['wall_s']:.0f} s (FP8 layer step {cpu['us_fp8_layer_step']:.0f} us)")

    full = {"metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
            "warmup": a.warmup, "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp8e4m3 weights x bf16 activations, fp32 accumulate",
            "data": "synthetic (seeded N(0,0.02) weights quantised to e4m3fn; N(0,1) bf16 x)",
            "config": {"workload": "FP8 W8A16 GEMV, M=1, Llama-3.1-8B layer: qkv 6144x4096, o 4096x4096, "
                                   "gate_up 28672x4096, down 4096x14336 (BASELINE configs[1])",
                       "layer_copies": L, "rotation_bytes": L * layer_bytes, "step_bytes": step_bytes,
                       "us_per_layer_step": round(ms_per_step * 1e3, 3),
                       "pct_of_8TBps": round(100 * value / PEAK_GBPS, 1), "timed_graph_primed": True},
            "roofline": roof, "roofline_by_dtype": by_dtype, "per_gemv": per, "b0": b0, "chain": chain,
            "cpu_baseline": cpu, "device": props.name, "cus": props.multi_processor_count,
            "timed_wall_ms": round(wall_ms, 3)}
    if a.report:
        Path(a.report).parent.mkdir(parents=True, exist_ok=True)
        Path(a.report).write_text(json.dumps(full, indent=1))
    print(json.dumps(compact_line(full, a.report)), flush=True)
    return 0


# roofline fields kept in the one-line record (the rest is in the report)
_ROOF_KEYS = ("bound", "achieved", "peak", "unit", "frac", "traffic", "kernel", "case", "avg_launch_us",
              "algorithmic_bytes")


def compact_line(full: dict, report: str | None = None) -> dict:
    """The driver's one JSON line from the full record: the contract keys, the dominant kernel's roofline, a
    three-entry roofline_by_dtype, per_gemv as {case: [us, % of 8 TB/s, over I/O floor]}, B0, the two decode chains
    as [us per token-step, GB/s, % of 8 TB/s] and a summary of the CPU baseline. Kept under 4 KB so the driver's
    output window holds it whole (the reference keeps one compact record per cell, paia-bench/bench/run.py:586-608)."""
    out = {k: full[k] for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config")}
    roof = full.get("roofline")
    out["roofline"] = None
    if roof:
        out["roofline"] = {k: roof.get(k) for k in _ROOF_KEYS}
        td = roof.get("traffic_detail") or {}
        out["roofline"]["traffic_over_algorithmic"] = td.get("over_algorithmic")
    out["roofline_by_dtype"] = {f: {"case": r["case"], "us": r["avg_launch_us"], "achieved": r["achieved"],
                                    "frac": r["frac"], "traffic": r["traffic"]}
                                for f, r in (full.get("roofline_by_dtype") or {}).items()}
    out["per_gemv"] = {n: [e["us"], e["pct_of_8TBps"], e.get("over_io_floor")]
                       for n, e in (full.get("per_gemv") or {}).items()}
    b0 = full.get("b0")
    out["b0"] = {"gbps": b0["gbps"], "pct_of_8TBps": b0["pct_of_8TBps"]} if b0 else None
    ch = full.get("chain")
    out["chain"] = {f: [c["us_per_token_step"], c["gbps"], c["pct_of_8TBps"]] for f, c in ch.items()} if ch else None
    cpu = full.get("cpu_baseline")
    out["cpu_baseline"] = None
    if cpu:
        out["cpu_baseline"] = {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample", "cpu",
                                                   "us_fp8_layer_step", "us_fp8_layer_step_matmul_only")}
        out["cpu_baseline"]["gemvs_timed"] = len(cpu.get("per_config", []))
    out["report"] = report
    return out


if __name__ == "__main__":
    sys.exit(main())
