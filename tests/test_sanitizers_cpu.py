"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU:

* the CPU oracle (oracle/w8a8_oracle.c, built with gcc) driven on small
  inputs in exactly sized heap buffers (sanitize_oracle_main.c);
* libw8a8.so's host code (the C ABI's validation and size queries, the GEMM,
  stream-K and MoE planners) built with each `-fsanitize=` behind
  `-Xarch_host`, so only the host pass is instrumented, and driven through
  every entry point's rejection paths and size queries
  (sanitize_capi_main.cpp; no call reaches a kernel launch);
* the two schedule brute-force checks (streamk_plan_check.cpp,
  moe_plan_check.cpp), host pass instrumented.

Any report (an out-of-bounds access, a use after free, a signed overflow, an
invalid shift or conversion) aborts the program and fails the test.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HERE = ROOT / "tests"
CSRC = ROOT / "optimized_rocwmma_samples_amd" / "csrc"

SAN = ["-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=all",
       "-fno-omit-frame-pointer"]
# host pass only: every sanitizer flag behind -Xarch_host on a hipcc line
HOST_SAN = [f for s in SAN for f in ("-Xarch_host", s)]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")


def _hipcc() -> str:
    h = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(h).exists():
        pytest.skip("hipcc not available")
    return h


def _run(cmd, timeout=600, env=None):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=timeout, env=env)
    return r.returncode, r.stdout


def test_oracle_under_sanitizers(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "sanitize_oracle"
    rc, out = _run([gcc, "-std=c11", "-O1", "-g", "-fopenmp", "-ffp-contract=off",
                    "-march=x86-64-v3", *SAN, str(HERE / "sanitize_oracle_main.c"),
                    str(ROOT / "oracle" / "w8a8_oracle.c"), "-o", str(exe), "-lm"])
    assert rc == 0, out[-3000:]
    rc, out = _run([str(exe)], env=dict(ENV, OMP_NUM_THREADS="4"))
    assert rc == 0 and out.strip().endswith("OK"), out[-4000:]


SOURCES = ["capi.cpp", "smoothquant.hip", "gemm_i8.hip", "moe.hip", "rmsnorm_sq.hip",
           "weights.hip"]


def test_capi_host_code_under_sanitizers(tmp_path):
    import concurrent.futures as cf
    hipcc = _hipcc()
    flags = ["-std=c++17", "-O1", "-g", "--offload-arch=gfx950", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             f"-I{ROOT / 'include'}", *HOST_SAN]

    def compile_one(src):
        obj = tmp_path / (Path(src).stem + ".o")
        return obj, _run([hipcc, "-x", "hip", *flags, "-c", str(CSRC / src), "-o", str(obj)])

    with cf.ThreadPoolExecutor(max_workers=min(6, os.cpu_count() or 2)) as ex:
        results = list(ex.map(compile_one, SOURCES))
    for obj, (rc, out) in results:
        assert rc == 0, out[-3000:]
    lib = tmp_path / "libw8a8_san.so"
    rc, out = _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *HOST_SAN,
                    "-shared-libsan", "-o", str(lib), *(str(o) for o, _ in results)])
    assert rc == 0, out[-3000:]
    exe = tmp_path / "sanitize_capi"
    # the shared sanitizer runtime lives in the compiler's resource directory
    rc, res = _run([hipcc, "-print-resource-dir"])
    assert rc == 0, res
    rt = Path(res.strip().splitlines()[-1]) / "lib" / "linux"
    rc, out = _run([hipcc, "-x", "hip", "--offload-host-only", "-std=c++17", "-O1", "-g",
                    f"-I{ROOT / 'include'}", *HOST_SAN, "-shared-libsan",
                    str(HERE / "sanitize_capi_main.cpp"), "-o", str(exe), f"-L{tmp_path}",
                    "-lw8a8_san", f"-Wl,-rpath,{tmp_path}", f"-Wl,-rpath,{rt}"])
    assert rc == 0, out[-3000:]
    rc, out = _run([str(exe)], env=ENV)
    assert rc == 0 and "OK" in out, out[-4000:]


@pytest.mark.parametrize("src", ["streamk_plan_check.cpp", "moe_plan_check.cpp"])
def test_plan_checks_under_sanitizers(tmp_path, src):
    hipcc = _hipcc()
    exe = tmp_path / Path(src).stem
    rc, out = _run([hipcc, "-std=c++17", "-O1", "-g", "--offload-arch=gfx950", *HOST_SAN,
                    str(HERE / src), "-o", str(exe)])
    assert rc == 0, out[-3000:]
    # the MoE check's random cases cut to 100 (of 800): instrumented, all
    # of them take about 90 s
    args = ["100"] if src.startswith("moe") else []
    rc, out = _run([str(exe), *args], env=ENV, timeout=900)
    assert rc == 0 and out.startswith("OK"), out[-4000:]
