"""rocprof_summary on small synthetic rocprofv3 CSV files: the kernel-trace
table, the counter averages with their derived MFMA / LDS metrics, and the
calibrated traffic lines that bench.py reads."""
from __future__ import annotations

import csv

import pytest

from optimized_rocwmma_samples_amd import rocprof_summary as R

GEMM = ("void w8a8::gemm::gemm_i8_persist_kernel<w8a8::gemm::Cfg<256, 256, 128, 2, 2, 4, 4, 16> >"
        "(w8a8::gemm::KArgs, int, int)")
NEG = "void at::native::vectorized_elementwise_kernel<4, at::native::neg_kernel_cuda>(int)"


def _write(path, fields, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        w.writerows(rows)


def _counters(path, kernel, grid, values, t0=1000, dur=100_000):
    fields = ["Dispatch_Id", "Grid_Size", "Kernel_Name", "Counter_Name", "Counter_Value",
              "Start_Timestamp", "End_Timestamp"]
    _write(path, fields, [{"Dispatch_Id": 1, "Grid_Size": grid, "Kernel_Name": kernel,
                           "Counter_Name": c, "Counter_Value": v, "Start_Timestamp": t0,
                           "End_Timestamp": t0 + dur} for c, v in values.items()])


def test_trace_table_compacts_names_and_averages(tmp_path):
    fields = ["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Start_Timestamp",
              "End_Timestamp"]
    _write(tmp_path / "t" / "run_kernel_trace.csv", fields,
           [{"Kernel_Name": GEMM, "Grid_Size_X": 131072, "Grid_Size_Y": 1, "Grid_Size_Z": 1,
             "Start_Timestamp": 0, "End_Timestamp": d} for d in (300_000, 500_000)])
    lines = R.trace(str(tmp_path / "t")).splitlines()
    assert len(lines) == 2
    assert lines[1].startswith("gemm_i8_persist_kernel<Cfg<256,256,128,2,2,4,4,16> >")
    cols = lines[1].split()
    assert cols[-4:] == ["131072", "2", "400.00", "300.00"]


def test_pmc_derived_metrics(tmp_path):
    # 100 us at 2 GHz: GUI_ACTIVE = 8 XCDs x 200000 cycles; MFMA busy half the
    # SIMD cycles; 1e9 units of 512 int8 ops
    _counters(tmp_path / "p" / "run_counter_collection.csv", GEMM, 131072,
              {"GRBM_GUI_ACTIVE": 8 * 200_000, "SQ_VALU_MFMA_BUSY_CYCLES": 1024 * 100_000,
               "SQ_LDS_IDX_ACTIVE": 5_120_000, "SQ_INSTS_VALU_MFMA_MOPS_I8": 1e9})
    out = R.pmc([str(tmp_path / "p")])
    assert ("mfma_busy_per_gui_cycle (MFMA_BUSY / (SIMDs x GUI_ACTIVE / XCDs); "
            "a lower bound) = 0.500") in out
    assert "clock" not in out
    assert "lds_active_per_mfma_busy_cycle = 0.050" in out
    assert f"lds_active_cycles_per_Mop_int8 = {5_120_000 / 512e3:.3f}" in out
    assert f"int8_TOPS (MOPS_I8 x 512 / duration) = {1e9 * 512 / 100_000 / 1e3:.0f}" in out


def test_traffic_calibrates_on_the_copy(tmp_path):
    # the copy reads and writes 2^30 bytes; its counters read half / all of it
    for kind, cal, val in (("fetch", 2**30 / 1024 / 2, 1000.0), ("write", 2**30 / 1024, 250.0)):
        d = tmp_path / kind
        name = "FETCH_SIZE" if kind == "fetch" else "WRITE_SIZE"
        _counters(d / "a" / "run_counter_collection.csv", NEG, 1 << 30, {name: cal})
        _counters(d / "b" / "run_counter_collection.csv", GEMM, 131072, {name: val})
    out = R.traffic(str(tmp_path / "fetch"), str(tmp_path / "write")).splitlines()
    assert out[0].startswith("calibration fetch_factor=2.0000 write_factor=1.0000")
    line = [l for l in out if "persist" in l][0]
    assert line.endswith(f"bytes={(1000.0 * 2 + 250.0) * 1024:.0f}")


def test_traffic_needs_the_calibration_copy(tmp_path):
    for kind in ("fetch", "write"):
        name = "FETCH_SIZE" if kind == "fetch" else "WRITE_SIZE"
        _counters(tmp_path / kind / "run_counter_collection.csv", GEMM, 131072, {name: 1.0})
    with pytest.raises(SystemExit):
        R.traffic(str(tmp_path / "fetch"), str(tmp_path / "write"))


def test_traffic_by_dispatch_order(tmp_path):
    # three launches of one kernel and grid per step, two steps: one line per
    # position of the cycle, from the dispatches in Dispatch_Id order
    fields = ["Dispatch_Id", "Grid_Size", "Kernel_Name", "Counter_Name", "Counter_Value"]
    for kind, name, cal, vals in (("fetch", "FETCH_SIZE", 2**30 / 1024 / 2, (10., 20., 30.)),
                                  ("write", "WRITE_SIZE", 2**30 / 1024, (1., 2., 3.))):
        rows = [{"Dispatch_Id": 1, "Grid_Size": 1 << 30, "Kernel_Name": NEG, "Counter_Name": name,
                 "Counter_Value": cal}]
        # written out of order: the summary sorts by Dispatch_Id
        for d in (7, 2, 5, 3, 6, 4):
            rows.append({"Dispatch_Id": d, "Grid_Size": 131072, "Kernel_Name": GEMM,
                         "Counter_Name": name, "Counter_Value": vals[(d - 2) % 3] + (d >= 5)})
        _write(tmp_path / kind / "run_counter_collection.csv", fields, rows)
    out = R.traffic(str(tmp_path / "fetch"), str(tmp_path / "write"), cycle=3).splitlines()
    pos = [l for l in out if " pos=" in l]
    assert [l.split(" pos=")[1].split()[0] for l in pos] == ["0/3", "1/3", "2/3"]
    for i, l in enumerate(pos):
        f, w = (10. + 10 * i) + 0.5, (1. + i) + 0.5
        assert f"fetch_kib={f:.1f} write_kib={w:.1f} bytes={(f * 2 + w) * 1024:.0f}" in l
    # without a cycle, or for kernels the cycle pattern does not match: no pos lines
    assert not [l for l in R.traffic(str(tmp_path / "fetch"), str(tmp_path / "write")).splitlines()
                if " pos=" in l]
    assert not [l for l in R.traffic(str(tmp_path / "fetch"), str(tmp_path / "write"), cycle=3,
                                     cycle_match="tile").splitlines() if " pos=" in l]


def test_bench_reads_per_projection_traffic_from_the_profile():
    # the committed cfg3 profile lists the persistent kernel's dispatches by
    # launch position: qkv, o_proj and gate_up get their own traffic (their
    # algorithmic bytes differ by 5x), down its tile-kernel row
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    import bench
    projs = [dict(m=8192, k=k, n=n) for _, k, n in bench.LLAMA3_8B]
    avg, per, by_order = bench.profiled_traffic(projs, 256)
    assert by_order and len(per) == 4
    assert per[2] > per[0] > per[1] > 0  # gate_up > qkv > o_proj
    assert avg == pytest.approx(sum(per) / 4)


def test_step_positions_take_whole_steps_from_the_end(tmp_path):
    # a partial step first (one quantizer), then three steps of 2 launches:
    # the quantizer (10, 12, 14 us) and the GEMM (100, 90, 95 us)
    sq = "void w8a8::(anonymous namespace)::sq_stream_kernel<4, 2, 256, false, false>(int)"
    fields = ["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Start_Timestamp",
              "End_Timestamp"]
    rows, t = [], 0
    seq = [(sq, 99_000)] + [x for a, b in ((10_000, 100_000), (12_000, 90_000), (14_000, 95_000))
                             for x in ((sq, a), (GEMM, b))]
    for name, d in seq:
        rows.append({"Kernel_Name": name, "Grid_Size_X": 512, "Grid_Size_Y": 1,
                     "Grid_Size_Z": 1, "Start_Timestamp": t, "End_Timestamp": t + d})
        t += d + 1000
    _write(tmp_path / "s" / "run_kernel_trace.csv", fields, rows)
    lines = R.step(str(tmp_path / "s"), 2).splitlines()
    assert lines[1].split()[1].startswith("sq_stream_kernel<4,2,256,false,false>")
    assert lines[1].split()[-3:] == ["3", "12.00", "10.00"]
    assert lines[2].split()[1] == "gemm_i8_persist_kernel<Cfg<256,256,128,2,2,4,4,16>"
    assert lines[2].split()[-3:] == ["3", "95.00", "90.00"]
    assert lines[3] == "sum of medians: 107.0 us per step"
    # a cycle length that does not match the steps shows up as MIXED
    assert "MIXED" in R.step(str(tmp_path / "s"), 3)
