"""Timing on MI355X: hipEvent pairs around hipGraph replays of back-to-back launches, with operand rotation that
defeats the 256 MiB Infinity Cache (MALL).

Methodology follows paia-bench/bench/timing.py:18-173 (graph mode: R launches captured in one graph, events around
one replay, per-op time = elapsed / R; warmup by calls and wall time; median of samples), re-based for MI355X:
  * rotation is sized against the last-level cache (Infinity Cache, 256 MiB) instead of L2: consecutive uses of one
    operand copy are separated by >= factor * 256 MiB of other traffic (n_copies = max(2, ceil(factor*LLC/footprint)));
  * torch.cuda.CUDAGraph / torch.cuda.Event are hipGraph / hipEvent on ROCm; events are recorded on the stream the
    kernels are launched on (torch's current stream, which the ctypes calls use).
"""
from __future__ import annotations

import math
import statistics
import time

import torch

LLC_BYTES = 256 * 2 ** 20          # MI355X Infinity Cache
HBM_PEAK_GBPS = 8000.0             # MI355X HBM3E, published


def plan_rotation(footprint: int, factor: float = 4.0, llc: int = LLC_BYTES, mem_cap: int = 64 * 2 ** 30) -> dict:
    want = max(2, math.ceil(factor * llc / max(1, footprint)))
    fit = max(1, mem_cap // max(1, footprint))
    n = min(want, fit)
    return {"n_copies": n, "rotation_bytes": n * footprint, "llc_bytes": llc, "llc_safe": n * footprint >= factor * llc}


def capture(fn, warm: int = 2) -> torch.cuda.CUDAGraph:
    """Capture fn() (which launches on torch's current stream) into a graph, after warm-up calls on a side stream."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warm):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def replay_ms(g: torch.cuda.CUDAGraph, n: int) -> list:
    """n timed replays; hipEvents on the current stream (where graph.replay() launches)."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    torch.cuda.synchronize()
    for a, b in ev:
        a.record()
        g.replay()
        b.record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def stats(samples: list) -> dict:
    s = sorted(samples)
    n = len(s)
    q = lambda p: s[min(n - 1, max(0, round(p * (n - 1))))]
    mean = statistics.fmean(s)
    return {"median": statistics.median(s), "p5": q(0.05), "p95": q(0.95), "mean": mean,
            "cv": (statistics.pstdev(s) / mean) if n > 1 and mean > 0 else 0.0, "n": n}


# The reference harness's cell protocol (paia-bench/configs/shapes.yaml:72-80, paia-bench/bench/timing.py:111-172,
# paia-bench/bench/run.py:200-270): per allocation a warm-up of >= 20 calls and >= 200 ms, then
# clamp(sample_target / unit, 30, 300) timed units, where a cell's 1000 ms sample target is split over its 5
# allocations; R is sized on the first allocation and kept for the others; the cell's value is the median across
# allocations.
WARMUP_MIN_CALLS = 20
WARMUP_MIN_MS = 200.0
SAMPLES_MIN, SAMPLES_MAX = 30, 300
CELL_SAMPLE_TARGET_MS = 1000.0
ALLOCATIONS_PER_CELL = 5


def time_per_call_us(call, n_copies: int, target_ms: float = 5.0, samples: int | None = None,
                     warmup_ms: float = WARMUP_MIN_MS, warmup_calls: int = WARMUP_MIN_CALLS,
                     sample_target_ms: float = CELL_SAMPLE_TARGET_MS / ALLOCATIONS_PER_CELL, R: int | None = None,
                     r_max: int = 4000) -> dict:
    """Per-call microseconds of call(i) (launch on copy i): one graph of R back-to-back calls cycling the copies,
    R sized so a replay lasts >= target_ms (or the R given, e.g. the first allocation's, rounded to whole rotations);
    warm-up replays until both warmup_calls calls and warmup_ms have passed; then `samples` timed replays, or, when
    samples is None, clamp(sample_target_ms / replay time, 30, 300) of them; the median per call."""
    if R is None:
        # estimate from a short graph
        r0 = min(r_max, max(8, 2 * n_copies))
        g = capture(lambda: [call(j % n_copies) for j in range(r0)])
        est = statistics.median(replay_ms(g, 3)) * 1e3 / r0
        del g
        R = int(min(r_max, max(r0, math.ceil(target_ms * 1e3 / max(est, 1e-3)))))
    R = max(n_copies, (R // n_copies) * n_copies)                # whole rotations
    g = capture(lambda: [call(j % n_copies) for j in range(R)])
    t0, calls = time.perf_counter(), 0
    while (time.perf_counter() - t0) * 1e3 < warmup_ms or calls < warmup_calls:
        g.replay()
        calls += R
    torch.cuda.synchronize()
    w_ms = (time.perf_counter() - t0) * 1e3
    if samples is None:
        unit_ms = statistics.median(replay_ms(g, 3))
        samples = int(min(SAMPLES_MAX, max(SAMPLES_MIN, math.ceil(sample_target_ms / max(unit_ms, 1e-3)))))
    ms = replay_ms(g, samples)
    del g
    per = [m * 1e3 / R for m in ms]
    st = stats(per)
    return {"us": st["median"], "R": R, "n_copies": n_copies, "warmup_calls": calls, "warmup_ms": round(w_ms, 1),
            **{f"us_{k}": v for k, v in st.items() if k != "median"}}
