"""HBM bytes per launch from rocprofv3 counters, calibrated on kernels of known size.

    # the workload, under the profiler (one counter pass per run: FETCH_SIZE, then WRITE_SIZE)
    rocprofv3 --pmc FETCH_SIZE -f csv -d OUT/fetch -o run -- python3 -m paia_bench.pmc run --fmt fp8 --shape 28672x4096
    rocprofv3 --pmc WRITE_SIZE -f csv -d OUT/write -o run -- python3 -m paia_bench.pmc run --fmt fp8 --shape 28672x4096
    # the per-dispatch summary that bench.py reports as roofline.traffic
    python3 -m paia_bench.pmc summarize --fetch OUT/fetch/run_counter_collection.csv \\
        --write OUT/write/run_counter_collection.csv --out profiles/pmc_traffic.json \\
        --case fp8_gate_up_28672x4096 --fmt fp8 --shape 28672x4096

    # every BASELINE GEMV in one process per counter pass (bench.py's cases, the library's picks):
    rocprofv3 --pmc FETCH_SIZE -f csv -d OUT/fetch -o run -- python3 -m paia_bench.pmc run --all --cases-out OUT/cases.json
    rocprofv3 --pmc WRITE_SIZE -f csv -d OUT/write -o run -- python3 -m paia_bench.pmc run --all --cases-out OUT/cases.json
    python3 -m paia_bench.pmc summarize --all --cases OUT/cases.json --fetch OUT/fetch/run_counter_collection.csv \
        --write OUT/write/run_counter_collection.csv --out profiles/pmc_traffic.json

`run` launches, eagerly and in this order: the streaming-read probe over exactly CAL_BYTES, the copy probe over
CAL_BYTES (reads CAL_BYTES, writes CAL_BYTES), then `reps` GEMVs of the named case rotating over enough operand
copies (>= 4 x 256 MiB) that every weight byte comes from HBM. `run --all` does the same for every BASELINE GEMV in
turn (one gated call, then `reps`) and writes the dispatch plan (case, kernel, GEMV dispatches) for `summarize --all`,
which assigns the profiled GEMV dispatches to the cases in order and checks each one's kernel name. FETCH_SIZE / WRITE_SIZE are reported by rocprofv3 in
KiB per dispatch; `summarize` divides each by what the same counter read for the calibration kernels (bytes counted
per byte moved), so `traffic` is in HBM bytes of the GEMV launch, next to its algorithmic bytes.

Why FETCH_SIZE needs the calibration on MI355X: rocprofv3 defines it for gfx950 as (TCC_BUBBLE*128 + (TCC_EA0_RDREQ -
TCC_BUBBLE - TCC_EA0_RDREQ_32B)*64 + TCC_EA0_RDREQ_32B*32) / 1024 KiB. On the read probe of 256 MiB, TCC_EA0_RDREQ
counts 2^21 requests (one per 128 bytes) while TCC_BUBBLE, the 128-byte request count, reads 0: every request is
weighed as 64 bytes, half its size, so FETCH_SIZE reads 0.5 byte per byte. An optional third pass of
TCC_EA0_RDREQ_DRAM_32B_sum (32-byte units, a 128-byte request counting 4) measures the bytes read from HBM
directly; it reads 1.0 per byte on the probe, with no calibration.
"""
from __future__ import annotations

import argparse
import csv
import json
import statistics
import sys
from pathlib import Path

CAL_BYTES = 256 * 2 ** 20


def _calibrate(P, cus, dev):
    """The calibration kernels: the streaming-read probe over exactly CAL_BYTES, then the copy probe (3 times each)."""
    import torch

    from paia_gemv.loader import current_raw_stream
    src = torch.empty(CAL_BYTES, dtype=torch.uint8, device=dev)
    dst = torch.empty(CAL_BYTES, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    src.random_(0, 255)
    torch.cuda.synchronize()
    for _ in range(3):
        if P.paia_probe_read(src.data_ptr(), CAL_BYTES, sink.data_ptr(), cus * 8, 1, current_raw_stream()):
            raise RuntimeError("read probe failed")
        if P.paia_probe_copy(src.data_ptr(), dst.data_ptr(), CAL_BYTES, cus * 8, current_raw_stream()):
            raise RuntimeError("copy probe failed")
    torch.cuda.synchronize()


def cmd_run_all(a) -> int:
    """Every BASELINE GEMV in turn: build its rotation, one call gated against the CPU reference, then `reps` calls."""
    import torch

    from paia_gemv import load_lib

    from .cases import BASELINE_GEMVS, GemvCase, case_name, kernel_name
    from .chain import sample_rows
    from .probe import load_probe
    from .timing import plan_rotation

    dev = torch.device("cuda:0")
    P = load_probe()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    _calibrate(P, cus, dev)
    lib = load_lib()
    plan = []
    for cfg, fmt, model, nm, N, K, bias in BASELINE_GEMVS:
        name = case_name(fmt, model, nm, N, K, bias)
        c = GemvCase(lib, fmt, N, K, bias=bias, name=name)
        n = plan_rotation(c.footprint())["n_copies"]
        c.build(n, dev, host_copy0=False)
        c.call(0)
        chk = c.check_copy(0, sample_rows(N, 64))
        if not chk["ok"]:
            raise RuntimeError(f"{name}: correctness gate failed: {chk}")
        for i in range(a.reps):
            c.call((i + 1) % n)
        torch.cuda.synchronize()
        plan.append({"case": name, "fmt": fmt, "N": N, "K": K, "bias": bias, "variant": c.variant,
                     "kernel": kernel_name(lib, fmt, c.variant, N, K), "dispatches": 1 + a.reps})
        print(f"pmc run: {name} variant {c.variant} {plan[-1]['kernel']} x{1 + a.reps} over {n} copies", flush=True)
        c.free()
        torch.cuda.empty_cache()
    if a.cases_out:
        Path(a.cases_out).parent.mkdir(parents=True, exist_ok=True)
        Path(a.cases_out).write_text(json.dumps(plan, indent=1))
    return 0


def cmd_run(a) -> int:
    import torch

    from paia_gemv import load_lib

    from .cases import GemvCase
    from .probe import load_probe
    from .timing import plan_rotation

    dev = torch.device("cuda:0")
    P = load_probe()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    _calibrate(P, cus, dev)
    lib = load_lib()
    N, K = map(int, a.shape.split("x"))
    if a.batch:
        case = GemvCase(lib, a.fmt, N, K, bias=a.bias, variant=a.variant, mode="batch", M=a.batch)
    else:
        case = GemvCase(lib, a.fmt, N, K, bias=a.bias, variant=a.variant)
    n = plan_rotation(case.footprint())["n_copies"]
    case.build(n, dev)
    chk = case.check(rows=list(range(min(N, 64))))
    if not chk["ok"]:
        raise RuntimeError(f"correctness gate failed: {chk}")
    for i in range(a.reps):
        case.call(i % n)
    torch.cuda.synchronize()
    print(f"pmc run: {a.fmt} {N}x{K} variant {case.variant} x{a.reps} over {n} copies; "
          f"algorithmic bytes {case.bytes()['total']}", flush=True)
    return 0


def _gemv_dispatches(path: Path, counter: str) -> list:
    """[(short kernel name, counter value)] of the GEMV dispatches of a counter CSV, in dispatch order."""
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name") != counter or "paia::gemv" not in r["Kernel_Name"]:
                continue
            rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"].split("(")[0].replace("void ", ""),
                         float(r["Counter_Value"])))
    return [(k, v) for _, k, v in sorted(rows)]


def _per_kernel(path: Path, counter: str) -> dict:
    """{short kernel name: [per-dispatch counter value, ...]} from a rocprofv3 counter_collection CSV."""
    out: dict = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name") != counter:
                continue
            name = r["Kernel_Name"]
            short = ("read_probe" if "read_probe_kernel" in name else "copy_probe" if "copy_probe_kernel" in name
                     else name.split("(")[0].replace("void ", "") if "paia::gemv" in name else None)
            if short is None:
                continue
            out.setdefault(short, []).append(float(r["Counter_Value"]))
    return out


def cmd_summarize(a) -> int:
    """Merge one profiled case into the summary file: {"calibration": ..., "cases": {name: {...}}}."""
    from paia_gemv.shapes import gemv_bytes

    fetch = _per_kernel(Path(a.fetch), "FETCH_SIZE")
    write = _per_kernel(Path(a.write), "WRITE_SIZE")
    dram = _per_kernel(Path(a.dram), "TCC_EA0_RDREQ_DRAM_32B_sum") if a.dram else None
    kib = 1024.0
    cal_read = statistics.median(fetch["read_probe"]) * kib / CAL_BYTES          # counted bytes per byte read
    cal_copy_r = statistics.median(fetch["copy_probe"]) * kib / CAL_BYTES
    cal_copy_w = statistics.median(write["copy_probe"]) * kib / CAL_BYTES        # counted bytes per byte written
    gemv = [k for k in fetch if not k.endswith("probe")]
    if len(gemv) != 1:
        raise SystemExit(f"expected one GEMV kernel in the trace, found {gemv}")
    k = gemv[0]
    N, K = map(int, a.shape.split("x"))
    fb = statistics.median(fetch[k]) * kib / cal_read
    wb = statistics.median(write.get(k, [0.0])) * kib / cal_copy_w
    out = Path(a.out)
    res = json.loads(out.read_text()) if out.exists() else {}
    res["calibration"] = {"bytes": CAL_BYTES, "fetch_per_byte_read_probe": round(cal_read, 4),
                          "fetch_per_byte_copy_probe": round(cal_copy_r, 4),
                          "write_per_byte_copy_probe": round(cal_copy_w, 4)}
    alg = gemv_bytes(a.fmt, N, K, a.bias)["total"]
    entry = {"kernel": k, "dispatches": len(fetch[k]), "fetch_bytes": round(fb), "write_bytes": round(wb),
             "traffic_bytes": round(fb + wb), "algorithmic_bytes": alg,
             "traffic_over_algorithmic": round((fb + wb) / alg, 4)}
    if dram is not None:
        # DRAM read requests in 32-byte units (a 128-byte request counts 4): bytes read from HBM, no calibration
        cal_dram = statistics.median(dram["read_probe"]) * 32.0 / CAL_BYTES
        res["calibration"]["dram32_bytes_per_byte_read_probe"] = round(cal_dram, 4)
        db = statistics.median(dram[k]) * 32.0
        entry["dram_read_bytes"] = round(db)
        entry["dram_read_over_algorithmic"] = round(db / alg, 4)
    res.setdefault("cases", {})[a.case] = entry
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(res, indent=1) + "\n")
    print(json.dumps(res["cases"][a.case] | {"calibration": res["calibration"]}, indent=1))
    return 0


def cmd_summarize_all(a) -> int:
    """Every case of a `run --all` plan into the summary file (entries replaced, others kept)."""
    from paia_gemv.shapes import gemv_bytes

    plan = json.loads(Path(a.cases).read_text())
    kib = 1024.0
    probes_f = _per_kernel(Path(a.fetch), "FETCH_SIZE")
    probes_w = _per_kernel(Path(a.write), "WRITE_SIZE")
    cal_read = statistics.median(probes_f["read_probe"]) * kib / CAL_BYTES
    cal_copy_r = statistics.median(probes_f["copy_probe"]) * kib / CAL_BYTES
    cal_copy_w = statistics.median(probes_w["copy_probe"]) * kib / CAL_BYTES
    passes = {"fetch": _gemv_dispatches(Path(a.fetch), "FETCH_SIZE"),
              "write": _gemv_dispatches(Path(a.write), "WRITE_SIZE")}
    if a.dram:
        probes_d = _per_kernel(Path(a.dram), "TCC_EA0_RDREQ_DRAM_32B_sum")
        passes["dram"] = _gemv_dispatches(Path(a.dram), "TCC_EA0_RDREQ_DRAM_32B_sum")
    want = sum(e["dispatches"] for e in plan)
    for k, rows in passes.items():
        if len(rows) != want:
            raise SystemExit(f"{k} pass: {len(rows)} GEMV dispatches, the plan has {want}")
    out = Path(a.out)
    res = json.loads(out.read_text()) if out.exists() else {}
    res["calibration"] = {"bytes": CAL_BYTES, "fetch_per_byte_read_probe": round(cal_read, 4),
                          "fetch_per_byte_copy_probe": round(cal_copy_r, 4),
                          "write_per_byte_copy_probe": round(cal_copy_w, 4)}
    if a.dram:
        res["calibration"]["dram32_bytes_per_byte_read_probe"] = round(
            statistics.median(probes_d["read_probe"]) * 32.0 / CAL_BYTES, 4)
    at = 0
    for e in plan:
        sl = {k: rows[at:at + e["dispatches"]] for k, rows in passes.items()}
        at += e["dispatches"]
        for k, rows in sl.items():
            names = {n for n, _ in rows}
            if names != {e["kernel"]}:
                raise SystemExit(f"{e['case']}: {k} pass dispatches run {names}, the plan names {e['kernel']}")
        # the first dispatch of each case is its gated call on copy 0: counted with the rest (same kernel, same bytes)
        fb = statistics.median(v for _, v in sl["fetch"]) * kib / cal_read
        wb = statistics.median(v for _, v in sl["write"]) * kib / cal_copy_w
        alg = gemv_bytes(e["fmt"], e["N"], e["K"], e["bias"])["total"]
        entry = {"kernel": e["kernel"], "dispatches": e["dispatches"], "fetch_bytes": round(fb),
                 "write_bytes": round(wb), "traffic_bytes": round(fb + wb), "algorithmic_bytes": alg,
                 "traffic_over_algorithmic": round((fb + wb) / alg, 4)}
        if a.dram:
            db = statistics.median(v for _, v in sl["dram"]) * 32.0
            entry["dram_read_bytes"] = round(db)
            entry["dram_read_over_algorithmic"] = round(db / alg, 4)
        res.setdefault("cases", {})[e["case"]] = entry
        print(f"{e['case']}: {e['kernel']} traffic/algorithmic {entry['traffic_over_algorithmic']}"
              + (f", DRAM read/algorithmic {entry['dram_read_over_algorithmic']}" if a.dram else ""))
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(res, indent=1) + "\n")
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    r.add_argument("--fmt", default="fp8", choices=["bf16", "fp8", "int4", "int4zp"])
    r.add_argument("--shape", default="28672x4096")
    r.add_argument("--variant", type=int, default=None)
    r.add_argument("--bias", action="store_true")
    r.add_argument("--reps", type=int, default=20)
    r.add_argument("--batch", type=int, default=0, help="M > 0: the small-batch kernels with M activation rows")
    r.add_argument("--all", action="store_true", help="every BASELINE GEMV in turn (bench.py's cases)")
    r.add_argument("--cases-out", default=None, help="--all: write the dispatch plan here")
    s = sub.add_parser("summarize")
    s.add_argument("--all", action="store_true", help="every case of a `run --all` plan (--cases)")
    s.add_argument("--cases", default=None, help="--all: the dispatch plan `run --all` wrote")
    s.add_argument("--fetch", required=True)
    s.add_argument("--write", required=True)
    s.add_argument("--dram", default=None, help="counter CSV of TCC_EA0_RDREQ_DRAM_32B_sum (optional)")
    s.add_argument("--out", required=True)
    s.add_argument("--case", default=None, help="name the entry is stored under (bench.py's case name)")
    s.add_argument("--fmt", default="fp8", choices=["bf16", "fp8", "int4", "int4zp"])
    s.add_argument("--shape", default="28672x4096")
    s.add_argument("--bias", action="store_true")
    a = ap.parse_args(argv)
    if a.cmd == "run":
        return cmd_run_all(a) if a.all else cmd_run(a)
    if a.all:
        return cmd_summarize_all(a)
    if not a.case:
        ap.error("summarize: --case is required without --all")
    return cmd_summarize(a)


if __name__ == "__main__":
    sys.exit(main())
