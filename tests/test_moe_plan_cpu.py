"""The MoE tile schedule (MoeShape, moe_plan_of, moe_whole_tile in
gemm_i8_grouped_kernel.hpp) on the CPU: moe_plan_check.cpp includes the
kernel header itself, is built with hipcc's host pass and checks by brute
force that every W and C tile runs exactly once (split tiles once per
k-piece, only C tiles split), that each XCD takes its W tiles first and a
contiguous range of C tiles, and that the tiles cover every output of every
expert exactly once."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


def test_moe_plan_by_brute_force(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    exe = tmp_path / "moe_plan_check"
    build = subprocess.run([hipcc, "-std=c++17", "-O2", "--offload-arch=gfx950",
                            str(HERE / "moe_plan_check.cpp"), "-o", str(exe)],
                           stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                           timeout=300)
    assert build.returncode == 0, build.stdout[-3000:]
    run = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                         text=True, timeout=300)
    assert run.returncode == 0 and run.stdout.startswith("OK"), run.stdout[-3000:]
