#!/usr/bin/env python3
"""Benchmark of the paia_gemv hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--report PATH] [--no-cpu] [--no-chain] [--no-b0]

Workload (the metric's configuration): FP8 W8A16 M=1 GEMVs at the Llama-3.1-8B per-layer shapes
qkv 6144x4096, o 4096x4096, gate_up 28672x4096, down 4096x14336, OCP e4m3fn weights with a per-row fp32 scale, bf16
activations and outputs. One step = the four GEMVs of one decoder layer; steps rotate over L distinct layer copies
whose total (>= 4 x 256 MiB) defeats the Infinity Cache, so every weight byte comes from HBM. The timed region is one
hipGraph replay of K steps (that graph launched once, untimed, beforehand), bracketed by device synchronisation,
with all inputs resident in HBM. Each GEMV uses the library's per-shape variant (paia_gemv_pick_variant, the frozen MI355X
sweep in paia-project_amd/tuned/mi355x.json).

Printed: ONE JSON line (the driver's contract) with value = aggregate algorithmic GB/s of the step, plus
  per_gemv      us/GEMV, GB/s and % of 8 TB/s for each shape (graph of R back-to-back launches rotating over
                >= 4 x 256 MiB of copies of that shape alone)
  roofline      the dominant kernel (gate_up): algorithmic bytes / its average launch time (hipEvents on the launch
                stream, inside this run) vs 8 TB/s; traffic = HBM bytes per launch from the committed rocprofv3
                FETCH_SIZE/WRITE_SIZE summary (profiles/pmc_traffic.json), calibrated on kernels of known size
  b0            the streaming-read probe in the same run (the reference's measured-bandwidth denominator "B0"): the
                best rate of a 2 GiB read, and the read floor for each GEMV's byte count under the same cold-cache
                rotation; per_gemv then also carries % of B0 and the GEMV time over that floor (skipped with --no-b0)
  chain         BASELINE configs[4]: 32 layers x 4 GEMVs + bf16 lm_head as one hipGraph, INT4 (asymmetric g128) and
                FP8: us per token-step and aggregate GB/s (skipped with --no-chain)
  cpu_baseline  the CPU path (oracle dequantisation + torch fp32 matmul) on the host cores, on a bounded sample
Copy 0 of every operand set is checked against the CPU fp32 reference (torch dequantisation + matmul, the reference
harness's gate) before anything is timed. The CPU oracle is used only by the cpu_baseline leg, as the CPU path timed.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "paia-project_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "µs/GEMV + achieved HBM GB/s (% of 8 TB/s), Llama-3.1-8B shapes, batch 1"
PEAK_GBPS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def measure_b0(dev, cases, per: dict) -> dict:
    """B0 (the reference's measured streaming-read bandwidth, src/tests/gemv_bf16_check.cu:228-252) in this run: the
    best rate of a 2 GiB nontemporal read over a few launch shapes, then, for each GEMV case, the read floor for its
    byte count (reads of that size rotating over the 2 GiB buffer, back to back in one graph). Adds pct_of_b0 and
    over_read_floor (GEMV µs / floor µs) to each per_gemv entry."""
    import torch
    from paia_bench.probe import b0_large, b0_sized, load_probe

    P = load_probe()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    buf = torch.empty(2 * 2 ** 30, dtype=torch.uint8, device=dev)
    buf.random_(0, 255)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    gbps, cfg = b0_large(P, buf, sink, cus, configs=((4, 1), (8, 1), (8, 4), (16, 1), (16, 4)), log=lambda m: None)
    sized = {}
    for c in cases:
        r = b0_sized(P, buf, sink, cus, c.bytes()["total"])
        sized[c.name] = {"bytes": r["bytes"], "us": round(r["us"], 3), "gbps": round(r["gbps"], 1)}
        e = per[c.name]
        e["pct_of_b0"] = round(100 * e["gbps"] / gbps, 1)
        e["over_read_floor"] = round(e["us"] / r["us"], 3)
    del buf
    torch.cuda.empty_cache()
    return {"gbps": round(gbps, 1), "pct_of_8TBps": round(100 * gbps / PEAK_GBPS, 1), "bytes": 2 * 2 ** 30,
            "blocks_per_cu": cfg[0], "unroll": cfg[1], "read_floor": sized}


def cpu_baseline(oracle, cases, budget_s: float = 12.0) -> dict:
    """The reference's CPU path (dequantise, then an fp32 matmul): the oracle's C dequantiser
    (one thread) and torch's CPU fp32 matmul on the host cores, over the layer's four shapes (seeded copy-0 operands)
    until ~budget_s."""
    import platform

    import torch
    from paia_bench.inputs import as_numpy

    threads = max(1, min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "64"))))
    torch.set_num_threads(threads)
    t_deq = t_mm = 0.0
    nbytes = 0
    steps = 0
    t_start = time.perf_counter()
    while True:
        for c in cases:
            a = as_numpy(c.ops0)
            t0 = time.perf_counter()
            Wd = oracle.dequant_fp8(a["Wq"], a["scale"])
            t1 = time.perf_counter()
            x = torch.from_numpy(oracle.bf16_bits_to_f32(a["x"]).copy())
            y = torch.from_numpy(Wd) @ x
            y = y.to(torch.bfloat16)
            t2 = time.perf_counter()
            t_deq += t1 - t0
            t_mm += t2 - t1
            nbytes += c.bytes()["total"]
            del Wd, y
        steps += 1
        if time.perf_counter() - t_start > budget_s or steps >= 20:
            break
    total = t_deq + t_mm
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        model = platform.processor()
    return {"value": round(nbytes / total / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{steps} layer step(s) x 4 FP8 GEMVs (Llama-3.1-8B qkv/o/gate_up/down, seeded copy 0): "
                      f"oracle C dequant (1 thread) + torch fp32 matmul ({threads} threads); "
                      f"us per layer step {total / steps * 1e6:.0f} (dequant {t_deq / steps * 1e6:.0f}, "
                      f"matmul {t_mm / steps * 1e6:.0f}); cpu {model}",
            "us_per_layer_step": round(total / steps * 1e6, 1),
            "matmul_only_gbps": round(nbytes / t_mm / 1e9, 3) if t_mm > 0 else None}


def load_traffic(case_name: str):
    """HBM bytes per launch of this GEMV case from the committed rocprofv3 PMC summary (profiles/pmc_traffic.json,
    written by `python -m paia_bench.pmc summarize`), or None if that case was not profiled."""
    f = ROOT / "profiles" / "pmc_traffic.json"
    if not f.exists():
        return None
    try:
        d = json.loads(f.read_text())
        e = d.get("cases", {}).get(case_name)
        return None if e is None else {"bytes": round(e["traffic_bytes"]), "kernel": e.get("kernel"),
                                       "fetch_bytes": round(e["fetch_bytes"]), "write_bytes": round(e["write_bytes"])}
    except (OSError, ValueError, KeyError):
        return None


def kernel_name(lib, case) -> str:
    """The template instance of gemv_kernel a case launches (as rocprofv3 names it)."""
    fam = {"bf16": lib.variants, "fp8": lib.variants_fp8}.get(case.fmt, lib.variants_int4)
    v = fam[case.variant]
    F = {"bf16": 0, "fp8": 1, "int4": 2, "int4zp": 3}[case.fmt]
    aux = (2 if v["S"] else 0) if case.fmt == "bf16" else 2
    return f"paia::gemv_kernel<{F}, {v['R']}, {v['U']}, {v['W']}, {aux}, {'true' if v['H'] else 'false'}>"


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--report", type=str, default=None, help="also write a detailed JSON report here")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-b0", action="store_true", help="skip the streaming-read probe (B0) leg")
    ap.add_argument("--no-chain", action="store_true", help="skip the decode-chain (configs[4]) measurement")
    a = ap.parse_args(argv)
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {a.gpus}). The M=1 GEMV shards along N "
              "with no collective (each GPU streams its N/g rows with the full x), so the one-GPU figure on one "
              "GPU's share is what this benchmark reports. Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch
    from paia_bench.cases import GemvCase
    from paia_bench.timing import LLC_BYTES, capture, plan_rotation, time_per_call_us
    from paia_gemv import load_lib
    from paia_gemv.shapes import LAYER

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (MI355X)", file=sys.stderr)
        return 3
    lib = load_lib()
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(0)
    log(f"device {props.name} CUs {props.multi_processor_count} lib {lib.path}")

    shapes = LAYER["llama31_8b"]
    cases = [GemvCase(lib, "fp8", N, K, name=f"fp8_{nm}_{N}x{K}") for nm, N, K in shapes]
    layer_bytes = sum(c.footprint() for c in cases)
    L = max(2, math.ceil(4 * LLC_BYTES / layer_bytes))
    for c in cases:
        c.build(L, dev)
    log(f"built {L} layer copies ({L * layer_bytes / 2**30:.2f} GiB); checking copy 0 against the CPU reference")
    for c in cases:
        chk = c.check()
        log(f"  {c.name}: variant {c.variant} rel_err {chk['rel_err']:.2e} ok {chk['ok']}")
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
    log(f"timed {a.steps} steps: {gpu_ms:.3f} ms (wall {wall_ms:.3f} ms), {ms_per_step * 1e3:.2f} us/step, "
        f"{value:.0f} GB/s")
    del g_warm, g_timed

    # per-GEMV figures: each shape on its own, rotating over enough copies of that shape alone (>= 4 x 256 MiB), so
    # the small shapes cannot run out of the Infinity Cache (the layer's L copies of one o_proj are only 84 MB)
    for c in cases:
        c.free()
    torch.cuda.empty_cache()
    per = {}
    for c in cases:
        n_rot = plan_rotation(c.footprint())["n_copies"]
        c.build(n_rot, dev)
        t = time_per_call_us(c.call, n_rot)
        c.free()
        torch.cuda.empty_cache()
        gbps = c.bytes()["total"] / (t["us"] * 1e-6) / 1e9
        per[c.name] = {"us": round(t["us"], 3), "gbps": round(gbps, 1), "pct_of_8TBps": round(100 * gbps / PEAK_GBPS, 1),
                       "variant": lib.variants_fp8[c.variant], "kernel": kernel_name(lib, c),
                       "bytes": c.bytes()["total"], "R": t["R"], "copies": n_rot}
        log(f"  {c.name}: {t['us']:.2f} us  {gbps:.0f} GB/s  ({100 * gbps / PEAK_GBPS:.1f}% of 8 TB/s)")

    dom = max(cases, key=lambda c: c.bytes()["total"])
    dom_us = per[dom.name]["us"]
    achieved = dom.bytes()["total"] / (dom_us * 1e-6) / 1e9
    traffic = load_traffic(dom.name)
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / PEAK_GBPS, 4), "traffic": traffic["bytes"] if traffic else None,
            "kernel": kernel_name(lib, dom), "case": dom.name, "avg_launch_us": dom_us,
            "algorithmic_bytes": dom.bytes()["total"],
            "traffic_detail": traffic}

    b0 = None
    if not a.no_b0:
        log("streaming-read probe (B0) ...")
        b0 = measure_b0(dev, cases, per)
        log(f"  b0 {b0['gbps']:.0f} GB/s ({b0['pct_of_8TBps']:.1f}% of 8 TB/s)")

    chain = None
    if not a.no_chain:
        from paia_bench.chain import run_chain
        log("decode chain (configs[4]) ...")
        chain = {f: run_chain(lib, f, log=log) for f in ("int4zp", "fp8")}

    cpu = None
    if not a.no_cpu:
        from oracle import oracle
        log("cpu baseline ...")
        from paia_bench.inputs import make_operands
        cpu_cases = [GemvCase(lib, "fp8", N, K, name=f"fp8_{nm}_{N}x{K}") for nm, N, K in shapes]
        for c in cpu_cases:
            c.ops0 = make_operands("fp8", c.N, c.K)
        cpu = cpu_baseline(oracle, cpu_cases)
        log(f"  cpu {cpu['value']:.2f} GB/s on {cpu['cores']} threads")

    out = {"metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
           "warmup": a.warmup, "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "fp8e4m3 weights x bf16 activations, fp32 accumulate",
           "data": "synthetic (seeded N(0,0.02) weights quantised to e4m3fn; N(0,1) bf16 x)",
           "config": {"workload": "FP8 W8A16 GEMV, M=1, Llama-3.1-8B layer: qkv 6144x4096, o 4096x4096, "
                                  "gate_up 28672x4096, down 4096x14336 (BASELINE configs[1])",
                      "layer_copies": L, "rotation_bytes": L * layer_bytes, "step_bytes": step_bytes,
                      "us_per_layer_step": round(ms_per_step * 1e3, 3),
                      "pct_of_8TBps": round(100 * value / PEAK_GBPS, 1), "timed_graph_primed": True},
           "per_gemv": per, "roofline": roof, "b0": b0, "chain": chain, "cpu_baseline": cpu}
    print(json.dumps(out), flush=True)
    if a.report:
        Path(a.report).parent.mkdir(parents=True, exist_ok=True)
        Path(a.report).write_text(json.dumps(out, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
