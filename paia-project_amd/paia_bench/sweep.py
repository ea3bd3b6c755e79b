"""Variant sweep on one MI355X: time every variant of a kernel family per shape and keep the fastest.

Counterpart of src/tools/dev_sweep_bf16.py:30-100 for gfx950: same idea (time each (R,U,W,S,H) tuple per N x K with
graph timing and rotation, keep the best and the top five), same tuned-table schema keyed "NxK" under "shapes" /
"fp8_shapes" / "int4_shapes" (paia-bench/bench/ops/ours_bf16.py:32-38, ours_quant.py:29-36).

    python -m paia_bench.sweep --fmt fp8 --shapes baseline --out OUT/sweep_fp8.json
    python -m paia_bench.sweep --fmt int4zp --shapes baseline --write-tuned paia-project_amd/tuned/mi355x.json
    python -m paia_bench.sweep --fmt fp8 --shapes baseline --batch 1,2,4,8,16     # small-batch kernels (P,U,W,S)
    python -m paia_bench.sweep --fmt fp8 --shapes frozen --candidates tuned --write-tuned paia-project_amd/tuned/mi355x.json
        (every other shape of the reference's frozen set, each timed with the variants that won a tuned shape)
    python -m paia_bench.sweep --fmt fp8 --merge rows.json mfma.json --write-tuned paia-project_amd/tuned/mi355x.json
        (small batch: the fastest measured variant per "MxNxK" over several sweeps' --out files)

Copy 0 of each shape is checked against the CPU fp32 reference (sampled rows) for every variant before it is timed.
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import numpy as np

from paia_gemv.shapes import LAYER, LM_HEAD, MODELS, SYNTHETIC

from .cases import GemvCase, kind_of
from .timing import HBM_PEAK_GBPS, plan_rotation, time_per_call_us

TKEY = {"bf16": "shapes", "fp8": "fp8_shapes", "int4": "int4_shapes", "int4zp": "int4_shapes"}


def shape_set(name: str, fmt: str):
    kmult = {"bf16": 8, "fp8": 16}.get(fmt, 128)
    out = []
    if name in ("baseline", "all"):
        for m in ("llama31_8b", "qwen25_7b"):
            out += [(f"{m}:{nm}", N, K) for nm, N, K in LAYER[m]]
        if fmt == "bf16":
            out += [(f"{m}:lm_head", *LM_HEAD[m]) for m in ("llama31_8b", "qwen25_7b")]
    if name in ("real", "all"):
        for m, shp in MODELS.items():
            out += [(f"{m}:{nm}", N, K) for nm, (N, K) in shp.items() if nm != "lm_head"]
    if name == "frozen":
        # the reference harness's frozen set (paia-bench/configs/shapes.yaml) minus the BASELINE shapes, which the
        # full sweep covers (a Qwen qkv entry there is timed with its bias)
        base = {(N, K) for _, N, K in shape_set("baseline", fmt)}
        for nm, (K, Ns) in SYNTHETIC.items():
            out += [(f"synthetic:{nm}_N{N}", N, K) for N in Ns if (N, K) not in base]
        for m, shp in MODELS.items():
            out += [(f"{m}:{nm}", N, K) for nm, (N, K) in shp.items() if (N, K) not in base]
    seen, uniq = set(), []
    for nm, N, K in out:
        if K % kmult == 0 and (N, K) not in seen:
            seen.add((N, K))
            uniq.append((nm, N, K))
    return uniq


def parse_filter(expr: str):
    import re
    conds = []
    for part in filter(None, (expr or "").split(",")):
        m = re.fullmatch(r"([RUWSHPX])(>=|<=|=)(\d+)", part.strip())
        if not m:
            raise SystemExit(f"bad filter term {part!r}")
        conds.append((m.group(1), m.group(2), int(m.group(3))))
    ops = {"=": lambda a, b: a == b, ">=": lambda a, b: a >= b, "<=": lambda a, b: a <= b}
    return lambda v: all(ops[o](v[k], n) for k, o, n in conds)


def main(argv=None):
    import torch

    from paia_gemv import load_lib

    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--fmt", choices=["bf16", "fp8", "int4", "int4zp"], required=True)
    ap.add_argument("--shapes", default="baseline", help="baseline | real | all | frozen | NxK[,NxK...]")
    ap.add_argument("--variants", default="", help="filter, e.g. 'R=2,U>=2,H=0'")
    ap.add_argument("--candidates", default="", help="'tuned': only the variants that are some shape's choice in "
                    "the tuned table (paia-project_amd/tuned/mi355x.json), plus the harness default")
    ap.add_argument("--target-ms", type=float, default=2.0)
    ap.add_argument("--samples", type=int, default=9)
    ap.add_argument("--out", default=None)
    ap.add_argument("--write-tuned", default=None)
    ap.add_argument("--batch", default="", help="M values: time the small-batch kernels (variants P,U,W,S,X)")
    ap.add_argument("--pick-only", action="store_true", help="time only the library's choice for each cell")
    ap.add_argument("--merge", nargs="+", default=None,
                    help="no timing: merge these --out files (fastest per cell) into --write-tuned")
    a = ap.parse_args(argv)
    if a.merge:
        if not a.write_tuned:
            raise SystemExit("--merge needs --write-tuned")
        merged = {}
        for fn in a.merge:
            for key, r in json.loads(Path(fn).read_text())["results"].items():
                if r["ranked"] and (key not in merged or r["ranked"][0]["us"] < merged[key]["ranked"][0]["us"]):
                    merged[key] = r
        write_tuned(Path(a.write_tuned), a.fmt, merged)
        return 0

    lib = load_lib()
    dev = torch.device("cuda:0")
    batch = [int(m) for m in a.batch.split(",") if m]
    if batch:
        fam = lib.variants_batch[a.fmt]
        knobs = "PUWSX"
    else:
        fam = {"bf16": lib.variants, "fp8": lib.variants_fp8}.get(a.fmt, lib.variants_int4)
        knobs = "RUWSH"
    keep = parse_filter(a.variants)
    if a.candidates == "tuned" and not batch:
        sec = TKEY[a.fmt] if a.fmt != "int4zp" else "int4zp_shapes"
        table = json.loads((Path(__file__).resolve().parent.parent / "tuned" / "mi355x.json").read_text())
        won = {tuple(e["variant"][k] for k in knobs) for e in table.get(sec, {}).values()}
        won.add({"bf16": (2, 4, 4, 0, 1), "fp8": (2, 2, 4, 0, 1)}.get(a.fmt, (4, 2, 4, 0, 1)))   # harness default
        filt = keep
        keep = lambda v: filt(v) and tuple(v[k] for k in knobs) in won
        have = set(table.get(sec, {}))         # shapes with a full-sweep entry keep it
    if a.shapes in ("baseline", "real", "all", "frozen"):
        shapes = shape_set(a.shapes, a.fmt)
    else:
        shapes = [(s, *map(int, s.split("x"))) for s in a.shapes.split(",")]
    if a.candidates == "tuned" and not batch:
        shapes = [(nm, N, K) for nm, N, K in shapes if f"{N}x{K}" not in have]
    cells = [(nm, N, K, M) for nm, N, K in shapes for M in (batch or [1])]
    results = {}
    for nm, N, K, M in cells:
        bias = a.fmt != "int4" and nm.endswith("qkv") and K == 3584
        if batch:
            case = GemvCase(lib, a.fmt, N, K, bias=bias, mode="batch", M=M)
        else:
            case = GemvCase(lib, a.fmt, N, K, bias=bias)
        rot = plan_rotation(case.footprint())
        t0 = time.time()
        case.build(rot["n_copies"], dev)
        rng = np.random.default_rng(0)
        rows = np.unique(np.concatenate([np.arange(min(N, 16)), N - 1 - np.arange(min(N, 16)),
                                         rng.integers(0, N, 64)])).astype(np.int32)
        tag = f"M={M} " if batch else ""
        print(f"[sweep] {a.fmt} {tag}{nm} {N}x{K}: {rot['n_copies']} copies, built in {time.time() - t0:.1f}s",
              flush=True)
        rows_res = []
        for v in fam:
            if not keep(v):
                continue
            if a.pick_only and v["id"] != case.variant:
                continue
            case.variant = v["id"]
            try:
                chk = case.check(rows=rows)
            except RuntimeError as e:            # batch: S*M*U too large for the LDS chunk (-2)
                print(f"  variant {v} refused: {e}", flush=True)
                continue
            if not chk["ok"]:
                print(f"  variant {v} INCORRECT {chk}", flush=True)
                continue
            t = time_per_call_us(case.call, rot["n_copies"], target_ms=a.target_ms, samples=a.samples,
                                 warmup_ms=20.0)
            gbps = case.bytes()["total"] / (t["us"] * 1e-6) / 1e9
            rows_res.append({"variant": {k: v[k] for k in knobs}, "id": v["id"], "us": t["us"], "gbps": gbps,
                             "cv": t.get("us_cv")})
            print("  " + " ".join(f"{k}={v[k]}" for k in knobs) + f": {t['us']:8.2f} us {gbps:7.0f} GB/s "
                  f"({100 * gbps / HBM_PEAK_GBPS:4.1f}%)", flush=True)
        rows_res.sort(key=lambda r: r["us"])
        key = f"{M}x{N}x{K}" if batch else f"{N}x{K}"
        results[key] = {"name": nm, "M": M, "bytes": case.bytes()["total"], "ranked": rows_res,
                        "pick": lib.batch_pick_variant(a.fmt, M, N, K) if batch else lib.pick_variant(a.fmt, N, K)}
        if rows_res:
            b = rows_res[0]
            print(f"[best] {a.fmt} {tag}{nm} {N}x{K}: {b['variant']} {b['us']:.2f} us {b['gbps']:.0f} GB/s "
                  f"({100 * b['gbps'] / HBM_PEAK_GBPS:.1f}% of 8 TB/s)", flush=True)
        case.free()
        torch.cuda.empty_cache()
        if a.out:   # rewritten after every cell, so a run stopped early keeps the cells it finished
            Path(a.out).parent.mkdir(parents=True, exist_ok=True)
            Path(a.out).write_text(json.dumps({"fmt": a.fmt, "results": results}, indent=1))
    if a.out:
        Path(a.out).parent.mkdir(parents=True, exist_ok=True)
        Path(a.out).write_text(json.dumps({"fmt": a.fmt, "results": results}, indent=1))
    if a.write_tuned:
        write_tuned(Path(a.write_tuned), a.fmt, results)
    return 0


def write_tuned(f: Path, fmt: str, results: dict):
    """Record each cell's fastest variant in the tuned table: M = 1 keys "NxK" under the reference's section names,
    small-batch keys "MxNxK" under "<fmt>_batch_shapes" ("batch_shapes" for BF16)."""
    tuned = json.loads(f.read_text()) if f.exists() else {"platform": "mi355x", "shapes": {}}
    for key, r in results.items():
        if not r["ranked"]:
            continue
        if key.count("x") == 2:
            sec = tuned.setdefault("batch_shapes" if fmt == "bf16" else f"{fmt}_batch_shapes", {})
        else:
            sec = tuned.setdefault(TKEY[fmt] if fmt != "int4zp" else "int4zp_shapes", {})
        best = r["ranked"][0]
        sec[key] = {"variant": best["variant"], "us": best["us"], "gbps": best["gbps"],
                    "top5": [{"variant": x["variant"], "pct_of_best": 100 * best["us"] / x["us"]}
                             for x in r["ranked"][:5]],
                    "when": time.strftime("%Y-%m-%d %H:%M")}
    f.parent.mkdir(parents=True, exist_ok=True)
    f.write_text(json.dumps(tuned, indent=1))


if __name__ == "__main__":
    sys.exit(main())
