"""Summarise a rocprofv3 kernel trace (``--kernel-trace -f csv``) per kernel and launch shape, as a markdown table.

    python3 -m paia_bench.rocprof_summary OUT/run_kernel_trace.csv [--pattern gemv_kernel]

Dispatches are grouped by (kernel name, grid in blocks, block size): the GEMV shapes that share one kernel
instantiation differ in their grid, so each row is one shape. Durations are End - Start of each dispatch (the
kernel's execution on the GPU, without the host-side launch).
"""
from __future__ import annotations

import argparse
import collections
import csv
import re
import statistics
import sys


def summarize(path: str, pattern: str = "paia") -> list[dict]:
    rows = collections.defaultdict(list)
    meta = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            if not re.search(pattern, name):
                continue
            name = re.sub(r"\(paia::GemvParams\)", "", name).replace("void ", "")
            wg = int(r["Workgroup_Size_X"]) if r.get("Workgroup_Size_X") else int(r["Workgroup_Size"])
            grid = int(r["Grid_Size_X"]) if r.get("Grid_Size_X") else int(r["Grid_Size"])
            key = (name, grid // max(1, wg), wg)
            rows[key].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
            meta[key] = {k: r.get(k, "") for k in ("VGPR_Count", "SGPR_Count", "LDS_Block_Size", "Scratch_Size")}
    out = []
    for key, d in sorted(rows.items(), key=lambda kv: -sum(kv[1])):
        d = sorted(d)
        out.append({"kernel": key[0], "blocks": key[1], "threads": key[2], "calls": len(d),
                    "avg_ns": statistics.fmean(d), "median_ns": d[len(d) // 2], "min_ns": d[0], **meta[key]})
    return out


def to_markdown(rows: list[dict]) -> str:
    lines = ["| kernel | blocks x threads | calls | avg ns | median ns | min ns | VGPR | SGPR | scratch |",
             "|---|---|---|---|---|---|---|---|---|"]
    for r in rows:
        lines.append(f"| `{r['kernel']}` | {r['blocks']} x {r['threads']} | {r['calls']} | {r['avg_ns']:.0f} | "
                     f"{r['median_ns']} | {r['min_ns']} | {r['VGPR_Count']} | {r['SGPR_Count']} | "
                     f"{r['Scratch_Size']} |")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("trace")
    ap.add_argument("--pattern", default="paia")
    a = ap.parse_args(argv)
    print(to_markdown(summarize(a.trace, a.pattern)))
    return 0


if __name__ == "__main__":
    sys.exit(main())
