"""The stream-K schedule's arithmetic (SkPlan, gemm_i8_streamk_kernel.hpp) on
the CPU: streamk_plan_check.cpp includes the kernel header itself, is built
with hipcc's host pass and checks coverage, piece counts and the partial
slots of every small (tiles, k-tiles, blocks) case by brute force."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


def test_streamk_plan_by_brute_force(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    exe = tmp_path / "streamk_plan_check"
    build = subprocess.run([hipcc, "-std=c++17", "-O2", "--offload-arch=gfx950",
                            str(HERE / "streamk_plan_check.cpp"), "-o", str(exe)],
                           stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                           timeout=300)
    assert build.returncode == 0, build.stdout[-3000:]
    run = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                         text=True, timeout=300)
    assert run.returncode == 0 and run.stdout.startswith("OK"), run.stdout[-3000:]
