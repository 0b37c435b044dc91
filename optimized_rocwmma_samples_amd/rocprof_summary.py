"""Summarize rocprofv3 CSV output for the W8A8 kernels.

    python -m optimized_rocwmma_samples_amd.rocprof_summary trace DIR        # kernel trace
    python -m optimized_rocwmma_samples_amd.rocprof_summary pmc DIR [DIR..]  # counters

Groups dispatches by (kernel, grid size) so the four projection GEMMs of one
bench step appear as separate rows, and prints per-dispatch averages.
"""
from __future__ import annotations

import csv
import glob
import os
import re
import sys
from collections import defaultdict


def short_name(name: str) -> str:
    name = re.sub(r"\(anonymous namespace\)::", "", name)
    m = re.match(r"(?:void )?([\w:]+(?:<[^()]*>)?)", name)
    base = m.group(1) if m else name[:80]
    return base.replace("w8a8::", "")


def _rows(pattern: str):
    for path in sorted(glob.glob(pattern, recursive=True)):
        with open(path, newline="") as f:
            yield from csv.DictReader(f)


def trace(directory: str, match: str = "w8a8|gemm|sq_|neg") -> str:
    groups = defaultdict(list)
    for r in _rows(os.path.join(directory, "**", "*kernel_trace.csv")):
        name = r.get("Kernel_Name", "")
        if not re.search(match, name):
            continue
        dur = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        grid = r.get("Grid_Size") or r.get("Grid_Size_X") or "?"
        groups[(short_name(name), grid)].append(dur)
    out = [f"{'kernel':60s} {'grid':>9s} {'calls':>5s} {'avg_us':>10s} {'min_us':>10s}"]
    for (name, grid), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"{name[:60]:60s} {grid:>9s} {len(d):5d} {sum(d) / len(d) / 1e3:10.2f} "
                   f"{min(d) / 1e3:10.2f}")
    return "\n".join(out)


def pmc(directories: list[str], match: str = "w8a8|gemm|sq_|neg") -> str:
    vals = defaultdict(lambda: defaultdict(list))
    for d in directories:
        for r in _rows(os.path.join(d, "**", "*counter_collection.csv")):
            name = r.get("Kernel_Name", "")
            if not re.search(match, name):
                continue
            key = (short_name(name), r.get("Grid_Size", "?"))
            vals[key][r["Counter_Name"]].append(float(r["Counter_Value"]))
    out = []
    for (name, grid), counters in sorted(vals.items()):
        out.append(f"{name} grid={grid}")
        for c, v in sorted(counters.items()):
            out.append(f"    {c:34s} dispatches={len(v):3d} avg={sum(v) / len(v):.6g}")
    return "\n".join(out)


def main(argv: list[str]) -> int:
    if len(argv) < 2 or argv[0] not in ("trace", "pmc"):
        print(__doc__)
        return 2
    if argv[0] == "trace":
        print(trace(argv[1]))
    else:
        print(pmc(argv[1:]))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
