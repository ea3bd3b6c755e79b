"""The reference harness's measurement phases, run against this library on one MI355X.

    python -m paia_bench.phases --phase s1,s3,s4 [--out results.json] [--quick] [--allocations 1] [--limit-mib N]

Cell sets (the frozen ones of paia-bench/bench/run.py:72-111 and src/patches/integration_quant.patch:9-60): every
synthetic shape (paia_gemv.shapes.SYNTHETIC) and every model shape (MODELS) at M = 1, in the three timing modes
  s1    BF16 GEMV (paia_gemv_bf16)
  s3    FP8 W8A16 GEMV (paia_gemv_fp8), shapes with K % 16 == 0
  s4    INT4 W4A16 g128: fused kernel in all modes; the naive (K1) and unfused controls in graph mode only
  s4zp  the asymmetric INT4 format of the BASELINE configs (paia_gemv_int4_zp), all modes  [no reference phase]
  e2    the platform library GEMM (torch.nn.functional.linear in bf16, i.e. hipBLASLt/rocBLAS) on the same cells,
        plus the model shapes at M = 2..16 in graph mode: the comparison the reference pairs s1 with
  sb    this library's small-batch kernels (paia_gemv_batch_*, FP8 and INT4 asym.) on the model shapes at the batch
        sweep's M, graph mode                                                                  [no reference phase]
Timing modes (paia-bench/bench/timing.py:1-6): isolated = one launch between device synchronisations; eager = events
around R back-to-back launches; graph = events around one replay of a graph of R launches. Per-op time = elapsed / R.
Rotation: each launch uses the next of n_copies operand sets, n_copies sized so two uses of one copy are >= 4 x 256 MiB
(the Infinity Cache) apart. Warm-up >= 20 calls and >= 200 ms, samples = clamp(1000 ms / unit, 30, 300), median per
allocation, median over allocations (paia-bench/configs/shapes.yaml:67-80). --quick shortens warm-up and sampling for
a smoke pass. Every (impl, shape) is gated on copy 0 against the CPU fp32 reference before it is timed (run.py:236-240).
"""
from __future__ import annotations

import argparse
import json
import math
import statistics
import sys
import time

import torch

from paia_gemv import load_lib
from paia_gemv.shapes import BATCH_M, MODELS, SYNTHETIC, gemv_bytes

from .cases import GemvCase
from .inputs import make_operands
from .timing import HBM_PEAK_GBPS, plan_rotation

FULL = {"warmup_min_calls": 20, "warmup_min_ms": 200.0, "samples_min": 30, "samples_max": 300,
        "sample_target_ms": 1000.0, "loop_target_ms": 5.0, "r_max": 20000}
QUICK = {**FULL, "warmup_min_ms": 30.0, "samples_min": 10, "samples_max": 60, "sample_target_ms": 150.0}
MODES = ("isolated", "eager", "graph")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ---- cells ---------------------------------------------------------------------------------------------------
def _m1_shapes(kmult: int):
    """(model, layer_name, N, K) of the frozen set with K % kmult == 0: synthetic sweep first, then model shapes."""
    out = []
    for name, (K, Ns) in SYNTHETIC.items():
        if K % kmult == 0:
            out += [("synthetic", f"{name}_N{N}", N, K) for N in Ns]
    for model, layers in MODELS.items():
        out += [(model, layer, N, K) for layer, (N, K) in layers.items() if K % kmult == 0]
    return out


def cells(phase: str) -> list:
    """The phase's cells: dicts with impl, fmt, mode (kernel family), M, N, K, model, layer_name, timing_mode."""
    def mk(impl, fmt, fam, model, layer, N, K, M, tmode):
        return {"phase": phase, "impl": impl, "fmt": fmt, "family": fam, "model": model, "layer_name": layer,
                "M": M, "N": N, "K": K, "timing_mode": tmode}
    out = []
    if phase == "s1":
        out = [mk("paia_gemv_bf16", "bf16", "fused", *s, 1, t) for s in _m1_shapes(8) for t in MODES]
    elif phase == "s3":
        out = [mk("paia_gemv_fp8", "fp8", "fused", *s, 1, t) for s in _m1_shapes(16) for t in MODES]
    elif phase == "s4":
        for s in _m1_shapes(128):
            out += [mk("paia_gemv_int4", "int4", "fused", *s, 1, t) for t in MODES]
            out.append(mk("paia_gemv_int4_naive", "int4", "naive", *s, 1, "graph"))
            out.append(mk("paia_gemv_int4_unfused", "int4", "unfused", *s, 1, "graph"))
    elif phase == "s4zp":
        out = [mk("paia_gemv_int4_zp", "int4zp", "fused", *s, 1, t) for s in _m1_shapes(128) for t in MODES]
    elif phase == "e2":
        out = [mk("torch_linear_bf16", "bf16", "library", *s, 1, t) for s in _m1_shapes(8) for t in MODES]
        for model, layers in MODELS.items():
            for layer, (N, K) in layers.items():
                out += [mk("torch_linear_bf16", "bf16", "library", model, layer, N, K, M, "graph")
                        for M in BATCH_M if M > 1]
    elif phase == "sb":
        for fmt in ("fp8", "int4zp"):
            for model, layers in MODELS.items():
                for layer, (N, K) in layers.items():
                    out += [mk(f"paia_gemv_batch_{fmt}", fmt, "batch", model, layer, N, K, M, "graph")
                            for M in BATCH_M]
    else:
        raise SystemExit(f"unknown phase {phase!r}")
    return out


# ---- the platform library GEMM as a case ---------------------------------------------------------------------
class LinearCase:
    """y = x @ W.T through torch.nn.functional.linear in bf16 (hipBLASLt / rocBLAS on ROCm): the library baseline
    the reference's e2 phase times (paia-bench/bench/ops/cublas_bf16.py). Same operands and gate as GemvCase."""

    def __init__(self, N, K, M=1):
        self.N, self.K, self.M, self.fmt, self.variant = N, K, M, "bf16", None
        self.copies, self.ops0 = [], None

    def bytes(self):
        return gemv_bytes("bf16", self.N, self.K, False, self.M)

    def footprint(self):
        return self.bytes()["total"]

    def build(self, n_copies, device="cuda", seed=1234):
        dev = torch.device(device)
        o = make_operands("bf16", self.N, self.K)
        gx = torch.Generator().manual_seed(2000 + self.M + self.N + self.K)
        xs = torch.randn(self.M, self.K, generator=gx).to(torch.bfloat16)
        xs[0] = o["x"]
        self.ops0 = {"W": o["W"], "x": xs}
        g = torch.Generator(device=dev).manual_seed(seed)
        self.copies = [(o["W"].to(dev), xs.to(dev))]
        for _ in range(n_copies - 1):
            self.copies.append(((0.02 * torch.randn(self.N, self.K, device=dev, generator=g)).to(torch.bfloat16),
                                torch.randn(self.M, self.K, device=dev, generator=g).to(torch.bfloat16)))
        return self

    def call(self, i, stream=None):
        W, x = self.copies[i]
        return torch.nn.functional.linear(x, W)

    def check(self, rtol=1e-2, atol=1e-2):
        y = self.call(0)
        torch.cuda.synchronize()
        y = y.cpu().float()
        ref = torch.empty(self.M, self.N)
        x = self.ops0["x"].float()
        for a in range(0, self.N, 8192):
            ref[:, a:a + 8192] = x @ self.ops0["W"][a:a + 8192].float().t()
        refb = ref.to(torch.bfloat16).float()
        excess = ((y - refb).abs() - (atol + rtol * refb.abs())).max().item()
        rel = ((y - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()
        ok = bool(torch.isfinite(y).all().item()) and excess <= 0 and rel < 2e-2
        return {"ok": ok, "rel_err": rel, "worst_excess": excess}

    def free(self):
        self.copies = []


# ---- timing --------------------------------------------------------------------------------------------------
class _Unit:
    """What one timing sample covers in a mode: 1 launch (isolated), R launches (eager), one replay of R (graph)."""

    def __init__(self, case, n, mode, R):
        self.case, self.n, self.mode, self.R, self.i, self.g = case, n, mode, R, 0, None
        if mode == "graph":
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for j in range(min(3, R)):
                    case.call(j % n)
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            self.g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.g):
                for j in range(R):
                    case.call(j % n)
            torch.cuda.synchronize()

    def _next(self):
        i = self.i
        self.i = (i + 1) % self.n
        return i

    def run(self):
        if self.mode == "graph":
            self.g.replay()
        elif self.mode == "eager":
            for _ in range(self.R):
                self.case.call(self._next())
        else:
            self.case.call(self._next())

    def timed(self, k):
        """Per-op µs for k samples."""
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(k)]
        if self.mode == "isolated":
            for a, b in ev:
                i = self._next()
                torch.cuda.synchronize()
                a.record()
                self.case.call(i)
                b.record()
                b.synchronize()
            return [a.elapsed_time(b) * 1e3 for a, b in ev]
        torch.cuda.synchronize()
        for a, b in ev:
            a.record()
            self.run()
            b.record()
        torch.cuda.synchronize()
        return [a.elapsed_time(b) * 1e3 / self.R for a, b in ev]


def measure(case, n_copies, mode, cfg):
    """One allocation's measurement of one mode: per-op µs samples and their statistics."""
    est = statistics.median(_Unit(case, n_copies, "isolated", 1).timed(10))
    R = 1 if mode == "isolated" else max(1, math.ceil(cfg["loop_target_ms"] * 1e3 / max(est, 1e-3)))
    u = _Unit(case, n_copies, mode, R)
    if mode != "isolated":
        # the isolated estimate carries launch + sync overhead; re-size R from a measured unit (a few times at most)
        for _ in range(3):
            u.run()
            unit_ms = statistics.median(u.timed(3)) * R / 1e3
            if unit_ms >= 0.9 * cfg["loop_target_ms"] or R >= cfg["r_max"]:
                break
            R = min(cfg["r_max"], math.ceil(R * cfg["loop_target_ms"] / max(unit_ms, 1e-4)))
            u = _Unit(case, n_copies, mode, R)
    calls, t0 = 0, time.perf_counter()
    while calls < cfg["warmup_min_calls"] or (time.perf_counter() - t0) * 1e3 < cfg["warmup_min_ms"]:
        u.run()
        calls += R
        torch.cuda.synchronize()
    unit_ms = statistics.median(u.timed(3)) * R / 1e3
    k = int(min(cfg["samples_max"], max(cfg["samples_min"], math.ceil(cfg["sample_target_ms"] / max(unit_ms, 1e-3)))))
    s = sorted(u.timed(k))
    n = len(s)
    mean = statistics.fmean(s)
    cv = statistics.pstdev(s) / mean if n > 1 and mean > 0 else 0.0
    return {"median_us": statistics.median(s), "p5_us": s[round(0.05 * (n - 1))], "p95_us": s[round(0.95 * (n - 1))],
            "cv": cv, "n_samples": n, "R": R, "warmup_calls": calls}


# ---- runner --------------------------------------------------------------------------------------------------
def make_case(lib, c):
    if c["family"] == "library":
        return LinearCase(c["N"], c["K"], c["M"])
    return GemvCase(lib, c["fmt"], c["N"], c["K"], mode=c["family"], M=c["M"])


def run(phases, cfg, allocations=1, limit_bytes=None, device="cuda"):
    lib = load_lib()
    records = []
    todo = [c for p in phases for c in cells(p)]
    # group the modes of one (phase, impl, shape, M): one build (allocation) serves all of its modes
    groups = {}
    for c in todo:
        groups.setdefault((c["phase"], c["impl"], c["family"], c["model"], c["layer_name"], c["M"], c["N"], c["K"]),
                          []).append(c)
    log(f"{len(todo)} cells in {len(groups)} (impl, shape) groups")
    for gi, (key, cs) in enumerate(groups.items()):
        phase, impl, fam, model, layer, M, N, K = key
        case = make_case(lib, cs[0])
        if limit_bytes and case.footprint() > limit_bytes:
            continue
        rot = plan_rotation(case.footprint())
        per_mode = {c["timing_mode"]: [] for c in cs}
        gate = None
        for a in range(allocations):
            case.build(rot["n_copies"], device)
            if a == 0:
                gate = case.check()
                if not gate["ok"]:
                    log(f"  GATE FAILED {impl} {layer} M={M} {N}x{K}: {gate}")
                    case.free()
                    break
            for c in cs:
                per_mode[c["timing_mode"]].append(measure(case, rot["n_copies"], c["timing_mode"], cfg))
            case.free()
            torch.cuda.empty_cache()
        if not gate or not gate["ok"]:
            records += [{**c, "error": "correctness gate failed", "gate": gate} for c in cs]
            continue
        nbytes = case.footprint()
        for c in cs:
            ms = per_mode[c["timing_mode"]]
            med = statistics.median(m["median_us"] for m in ms)
            gbps = nbytes / (med * 1e-6) / 1e9
            records.append({**c, "variant": case.variant, "bytes": nbytes, "n_copies": rot["n_copies"],
                            "allocations": ms, "median_us": med, "gbps": gbps,
                            "pct_of_8TBps": 100.0 * gbps / HBM_PEAK_GBPS, "gate": gate})
        modes = " ".join(f"{c['timing_mode']} {records[-len(cs) + i]['median_us']:.2f}" for i, c in enumerate(cs))
        log(f"[{gi + 1}/{len(groups)}] {phase} {impl} {model}:{layer} M={M} {N}x{K}: {modes} us")
    return records


def summary(records) -> str:
    """Markdown: per phase and impl, one row per shape with the median µs (and % of 8 TB/s) of each timing mode."""
    out = []
    keyf = lambda r: (r["phase"], r["impl"])
    for (phase, impl) in sorted({keyf(r) for r in records}):
        rs = [r for r in records if keyf(r) == (phase, impl) and "median_us" in r]
        modes = [m for m in MODES if any(r["timing_mode"] == m for r in rs)]
        out.append(f"\n**{phase} {impl}**\n")
        out.append("| shape | M | N x K | " + " | ".join(f"{m} µs (% of 8 TB/s)" for m in modes) + " |")
        out.append("|---|---|---|" + "---|" * len(modes))
        rows = {}
        for r in rs:
            rows.setdefault((r["model"], r["layer_name"], r["M"], r["N"], r["K"]), {})[r["timing_mode"]] = r
        for (model, layer, M, N, K), d in rows.items():
            cellsx = [f"{d[m]['median_us']:.2f} ({d[m]['pct_of_8TBps']:.1f}%)" if m in d else "–" for m in modes]
            out.append(f"| {model}:{layer} | {M} | {N}x{K} | " + " | ".join(cellsx) + " |")
    return "\n".join(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--phase", default="s1,s3,s4", help="comma list of s1, s3, s4, s4zp, e2, sb")
    ap.add_argument("--out", default=None, help="write every record as JSON here")
    ap.add_argument("--summary", default=None, help="write the markdown summary here")
    ap.add_argument("--quick", action="store_true", help="short warm-up and sampling (a smoke pass)")
    ap.add_argument("--allocations", type=int, default=1, help="independent operand allocations per cell (ref: 5)")
    ap.add_argument("--limit-mib", type=float, default=None, help="skip shapes whose footprint exceeds this")
    a = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("paia_bench.phases needs a GPU", file=sys.stderr)
        return 3
    cfg = QUICK if a.quick else FULL
    recs = run([p for p in a.phase.split(",") if p], cfg, a.allocations,
               None if a.limit_mib is None else int(a.limit_mib * 2 ** 20))
    text = summary(recs)
    print(text, flush=True)
    if a.out:
        with open(a.out, "w") as f:
            json.dump({"phases": a.phase, "timing": cfg, "allocations": a.allocations, "records": recs}, f, indent=1)
    if a.summary:
        with open(a.summary, "w") as f:
            f.write(text + "\n")
    bad = [r for r in recs if "error" in r]
    return 1 if bad else 0


if __name__ == "__main__":
    raise SystemExit(main())
