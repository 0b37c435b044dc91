"""Summarize rocprofv3 CSV output for the W8A8 kernels.

    python -m optimized_rocwmma_samples_amd.rocprof_summary trace DIR        # kernel trace
    python -m optimized_rocwmma_samples_amd.rocprof_summary pmc DIR [DIR..]  # counters
    python -m optimized_rocwmma_samples_amd.rocprof_summary traffic FETCH_DIR WRITE_DIR [CYCLE [REGEX]]
    python -m optimized_rocwmma_samples_amd.rocprof_summary step DIR LAUNCHES  # per launch of a step

`step` takes the traced W8A8 dispatches in start order as whole steps of
LAUNCHES launches each (the last whole steps of the run) and prints one line
per launch position of the step: kernel, grid, median and minimum duration
over the steps, then the sum of the medians.  A position whose dispatches are
not all one kernel prints MIXED (the trace does not hold whole steps).

`traffic` turns FETCH_SIZE and WRITE_SIZE (KiB per dispatch, one run each) into
bytes per dispatch, scaled by what the same counters read for the calibration
copy that `bench.py --calibrate-copy` runs (torch neg over 2^30 int8: 2^30
bytes read, 2^30 bytes written).  Output lines:
    traffic <kernel> grid=<g> fetch_kib=<f> write_kib=<w> bytes=<scaled total>

Groups dispatches by (kernel, grid size) so the four projection GEMMs of one
bench step appear as separate rows, and prints per-dispatch averages.  With
CYCLE (> 1), kernels matching REGEX (default "persist") whose dispatches of
one grid come in a repeating order of CYCLE launches (the persistent GEMM runs
qkv, o_proj, gate_up in every bench step, all with one block per CU) also get
one line per position in that order, from the dispatches in Dispatch_Id order:
    traffic <kernel> grid=<g> pos=<i>/<CYCLE> fetch_kib=<f> write_kib=<w> bytes=<b>
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


def compact_name(name: str) -> str:
    """short_name without the gemm:: namespace and the blanks after template
    argument commas, so kernels with two tile configurations fit a column."""
    return short_name(name).replace("gemm::", "").replace(", ", ",")


def _rows(pattern: str):
    for path in sorted(glob.glob(pattern, recursive=True)):
        with open(path, newline="") as f:
            yield from csv.DictReader(f)


def _grid(r: dict) -> str:
    """Total work-items of a dispatch: the kernel trace gives X, Y, Z apart
    (a 2-D launch such as a split-K grid would otherwise show only X)."""
    if r.get("Grid_Size"):
        return r["Grid_Size"]
    dims = [r.get(f"Grid_Size_{a}") for a in "XYZ"]
    if not dims[0]:
        return "?"
    total = 1
    for d in dims:
        total *= int(d) if d else 1
    return str(total)


def trace(directory: str, match: str = "w8a8|gemm|sq_|neg") -> str:
    groups = defaultdict(list)
    for r in _rows(os.path.join(directory, "**", "*kernel_trace.csv")):
        name = r.get("Kernel_Name", "")
        if not re.search(match, name):
            continue
        dur = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        groups[(compact_name(name), _grid(r))].append(dur)
    out = [f"{'kernel':88s} {'grid':>9s} {'calls':>5s} {'avg_us':>10s} {'min_us':>10s}"]
    for (name, grid), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"{name[:88]:88s} {grid:>9s} {len(d):5d} {sum(d) / len(d) / 1e3:10.2f} "
                   f"{min(d) / 1e3:10.2f}")
    return "\n".join(out)


def step(directory: str, launches: int, match: str = "w8a8|gemm|sq_") -> str:
    rows = [r for r in _rows(os.path.join(directory, "**", "*kernel_trace.csv"))
            if re.search(match, r.get("Kernel_Name", "")) and "peak" not in r.get("Kernel_Name", "")]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    whole = len(rows) // launches * launches
    rows = rows[len(rows) - whole:]
    out = [f"{'pos':>3s} {'kernel':82s} {'grid':>9s} {'steps':>5s} {'median_us':>10s} "
           f"{'min_us':>8s}"]
    total = 0.0
    for i in range(launches):
        at = rows[i::launches]
        names = {compact_name(r["Kernel_Name"]) for r in at}
        grids = {_grid(r) for r in at}
        d = sorted(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in at)
        med = d[len(d) // 2] / 1e3 if d else 0.0
        total += med
        name = names.pop() if len(names) == 1 else "MIXED"
        grid = grids.pop() if len(grids) == 1 else "MIXED"
        out.append(f"{i:3d} {name[:82]:82s} {grid:>9s} {len(d):5d} {med:10.2f} "
                   f"{(d[0] / 1e3 if d else 0.0):8.2f}")
    out.append(f"sum of medians: {total:.1f} us per step")
    return "\n".join(out)


def pmc(directories: list[str], match: str = "w8a8|gemm|sq_|neg") -> str:
    vals = defaultdict(lambda: defaultdict(list))
    durs = defaultdict(dict)  # dispatch id -> duration (ns), per kernel
    for d in directories:
        for r in _rows(os.path.join(d, "**", "*counter_collection.csv")):
            name = r.get("Kernel_Name", "")
            if not re.search(match, name):
                continue
            key = (short_name(name), r.get("Grid_Size", "?"))
            vals[key][r["Counter_Name"]].append(float(r["Counter_Value"]))
            if r.get("Start_Timestamp") and r.get("End_Timestamp"):
                durs[key][(d, r.get("Dispatch_Id"))] = (int(r["End_Timestamp"])
                                                        - int(r["Start_Timestamp"]))
    out = []
    for (name, grid), counters in sorted(vals.items()):
        out.append(f"{name} grid={grid}")
        avg = {c: sum(v) / len(v) for c, v in counters.items()}
        for c, v in sorted(counters.items()):
            out.append(f"    {c:34s} dispatches={len(v):3d} avg={avg[c]:.6g}")
        dur = list(durs[(name, grid)].values())
        out.extend("    " + line for line in _derived(avg, sum(dur) / len(dur) if dur else 0.0))
    return "\n".join(out)


# MI355X: 8 XCDs of 32 CUs, 4 SIMDs per CU.  GRBM_GUI_ACTIVE is summed over
# the XCDs; SQ_VALU_MFMA_BUSY_CYCLES over the SIMDs.
XCDS, SIMDS = 8, 1024


def _derived(avg: dict, dur_ns: float) -> list[str]:
    """Metrics derived from one kernel's averaged counters: MFMA-busy cycles
    per GPU-busy cycle, LDS-active cycles per MFMA-busy cycle and per int8
    op, and the int8 rate.

    GRBM_GUI_ACTIVE counts the GPU's busy cycles over the whole window the
    profiler brackets a dispatch with, launch and drain included, which is
    longer than the kernel's own run (for kernels of a few microseconds,
    several times longer), so MFMA_BUSY over it is a lower bound of the
    MFMA pipes' busy fraction, and GUI_ACTIVE over the trace's duration is
    not a clock: no clock is derived here."""
    out = []
    gui = avg.get("GRBM_GUI_ACTIVE")
    busy = avg.get("SQ_VALU_MFMA_BUSY_CYCLES")
    lds = avg.get("SQ_LDS_IDX_ACTIVE")
    mops = avg.get("SQ_INSTS_VALU_MFMA_MOPS_I8")
    if gui and busy is not None:
        out.append(f"mfma_busy_per_gui_cycle (MFMA_BUSY / (SIMDs x GUI_ACTIVE / XCDs); "
                   f"a lower bound) = {busy / (SIMDS * gui / XCDS):.3f}")
    if lds is not None and busy:
        out.append(f"lds_active_per_mfma_busy_cycle = {lds / busy:.3f}")
    if lds is not None and mops:
        out.append(f"lds_active_cycles_per_Mop_int8 = {lds / (mops * 512 / 1e6):.3f}")
    if mops and dur_ns > 0:
        out.append(f"int8_TOPS (MOPS_I8 x 512 / duration) = {mops * 512 / dur_ns / 1e3:.0f}")
    return out


CALIB_BYTES = 1 << 30
CALIB_KERNEL = "neg_kernel"


def _counter_avgs(directory: str, counter: str):
    vals = defaultdict(list)
    for r in _rows(os.path.join(directory, "**", "*counter_collection.csv")):
        if r["Counter_Name"] != counter:
            continue
        name = r.get("Kernel_Name", "")
        vals[(short_name(name), r.get("Grid_Size", "?"), name)].append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in vals.items()}


def _counter_seqs(directory: str, counter: str):
    """Per (kernel, grid): the counter's values in Dispatch_Id order."""
    vals = defaultdict(list)
    for r in _rows(os.path.join(directory, "**", "*counter_collection.csv")):
        if r["Counter_Name"] != counter:
            continue
        key = (short_name(r.get("Kernel_Name", "")), r.get("Grid_Size", "?"))
        vals[key].append((int(r.get("Dispatch_Id", 0)), float(r["Counter_Value"])))
    return {k: [v for _, v in sorted(d)] for k, d in vals.items()}


def traffic(fetch_dir: str, write_dir: str, match: str = "w8a8|gemm|sq_", cycle: int = 0,
            cycle_match: str = "persist") -> str:
    fetch = _counter_avgs(fetch_dir, "FETCH_SIZE")
    write = _counter_avgs(write_dir, "WRITE_SIZE")

    def calib(vals):
        # the calibration copy is the only elementwise launch over 2^30 elements
        cands = [v for (n, g, full), v in vals.items()
                 if CALIB_KERNEL in full and "elementwise" in full]
        if not cands:
            raise SystemExit("calibration copy not found (run bench.py --calibrate-copy)")
        return CALIB_BYTES / (cands[0] * 1024)

    ff, wf = calib(fetch), calib(write)
    out = [f"calibration fetch_factor={ff:.4f} write_factor={wf:.4f} "
           f"(torch neg over 2^30 int8 elements)"]
    wkeys = {(n, g): v for (n, g, _), v in write.items()}
    for (name, grid, full), f in sorted(fetch.items()):
        if not re.search(match, full):
            continue
        w = wkeys.get((name, grid), 0.0)
        total = (f * ff + w * wf) * 1024
        out.append(f"traffic {name.replace(' ', '')} grid={grid} fetch_kib={f:.1f} "
                   f"write_kib={w:.1f} bytes={total:.0f}")
    if cycle > 1:
        fseq, wseq = _counter_seqs(fetch_dir, "FETCH_SIZE"), _counter_seqs(write_dir, "WRITE_SIZE")
        for (name, grid), fs in sorted(fseq.items()):
            ws = wseq.get((name, grid), [])
            # each run is whole steps of its own (the two runs' step counts
            # may differ: the bench settles the clocks for a fixed time)
            if not re.search(cycle_match, name) or not ws or len(fs) % cycle or len(ws) % cycle:
                continue
            for i in range(cycle):
                f = sum(fs[i::cycle]) / len(fs[i::cycle])
                w = sum(ws[i::cycle]) / len(ws[i::cycle])
                out.append(f"traffic {name.replace(' ', '')} grid={grid} pos={i}/{cycle} "
                           f"fetch_kib={f:.1f} write_kib={w:.1f} bytes={(f * ff + w * wf) * 1024:.0f}")
    return "\n".join(out)


def main(argv: list[str]) -> int:
    if len(argv) < 2 or argv[0] not in ("trace", "pmc", "traffic", "step"):
        print(__doc__)
        return 2
    if argv[0] == "trace":
        print(trace(argv[1]))
    elif argv[0] == "step":
        if len(argv) != 3 or int(argv[2]) < 1:
            print(__doc__)
            return 2
        print(step(argv[1], int(argv[2])))
    elif argv[0] == "pmc":
        print(pmc(argv[1:]))
    else:
        if len(argv) not in (3, 4, 5):
            print(__doc__)
            return 2
        extra = {"cycle": int(argv[3])} if len(argv) > 3 else {}
        if len(argv) > 4:
            extra["cycle_match"] = argv[4]
        print(traffic(argv[1], argv[2], **extra))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
