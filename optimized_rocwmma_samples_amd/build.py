"""Build libw8a8.so (gfx950 HIP kernels + C ABI) and the C++ sample CLIs in-tree.

    python -m optimized_rocwmma_samples_amd.build [-g gfx950] [-t TARGET] [-j N] [-b DIR]
                                                  [-c] [-d] [-v] [--no-apps]
    optimized_rocwmma_samples_amd/build.sh        (the same options)

Every HIP translation unit is compiled with hipcc for gfx950 only.  The built
library lands in optimized_rocwmma_samples_amd/lib/, the CLIs in
optimized_rocwmma_samples_amd/bin/ (both git-ignored, both shipped with the
tree to the GPU box).  `--debug` builds the CLIs with the CPU-verify switch on (the default build
also puts debug builds of two CLIs in bin/debug/ for the GPU tests),
the reference's `build.sh -d` (build.sh:43, a Debug build
leaves NDEBUG undefined and enables the `#if !NDEBUG` check,
rocwmma_perf_gemm.cpp:736-749).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
APPS = PKG / "apps"
LIB_DIR = PKG / "lib"
BIN_DIR = PKG / "bin"
OBJ_DIR = PKG / "_build"
LIB_PATH = LIB_DIR / "libw8a8.so"
# measured-ceiling kernels timed by bench.py (not part of the W8A8 C ABI)
PEAKS_SRC = "peaks.hip"
PEAKS_PATH = LIB_DIR / "libw8a8_peaks.so"

ARCH = "gfx950"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

SOURCES = [
    "capi.cpp",
    "smoothquant.hip",
    "gemm_i8.hip",
    "moe.hip",
    "rmsnorm_sq.hip",
    "weights.hip",
]

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
HIP_FLAGS = [
    "-std=c++17",
    "-O3",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


def hipcc() -> str:
    cand = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    if not os.path.exists(cand):
        raise RuntimeError("hipcc not found; the W8A8 library needs ROCm's hipcc")
    return cand


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l
                    and "not a recognized feature" not in l and l.strip())
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}")
    if verbose and out:
        print(out)


def _compile(src: Path, obj: Path, verbose: bool, extra: list[str]) -> Path:
    lang = ["-x", "hip"] if src.suffix in (".hip", ".cpp") else []
    _run([hipcc(), *lang, *HIP_FLAGS, *extra, "-c", str(src), "-o", str(obj)], verbose)
    return obj


def build_library(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source for gfx950 and link lib/libw8a8.so."""
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, CSRC / s, OBJ_DIR / (Path(s).stem + ".o"), verbose, [])
                for s in SOURCES]
        for f in futs:
            objs.append(f.result())
    _link(LIB_PATH, objs, verbose)
    peaks = _compile(CSRC / PEAKS_SRC, OBJ_DIR / (Path(PEAKS_SRC).stem + ".o"), verbose, [])
    _link(PEAKS_PATH, [peaks], verbose)
    return LIB_PATH


def _link(path: Path, objs: list[Path], verbose: bool) -> None:
    tmp = path.with_suffix(".so.tmp")
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs)], verbose)
    os.replace(tmp, path)


def build_apps(debug: bool = False, verbose: bool = False, only: str | None = None,
               bin_dir: Path | None = None, jobs: int | None = None) -> list[Path]:
    """Build the reference-compatible sample CLIs against libw8a8.so (all of
    them, or the one named `only`) into `bin_dir` (default: the package's bin/)."""
    if not APPS.is_dir():
        return []
    out_dir = Path(bin_dir) if bin_dir else BIN_DIR
    out_dir.mkdir(parents=True, exist_ok=True)
    verify = ["-UNDEBUG", "-DW8A8_CPU_VERIFY=1"] if debug else ["-DNDEBUG"]
    srcs = sorted(APPS.glob("*.cpp"))
    if only is not None:
        srcs = [s for s in srcs if s.stem == only]
        if not srcs:
            raise RuntimeError(f"no sample named {only!r} (have: "
                               f"{', '.join(s.stem for s in sorted(APPS.glob('*.cpp')))})")

    def one(src: Path) -> Path:
        exe = out_dir / src.stem
        # host-only programs: no device code, so no offload target
        _run([hipcc(), "-x", "hip", "--offload-host-only", "-std=c++17", "-O3", "-Wall",
              f"-I{ROOT / 'include'}", *verify, "-fopenmp", str(src), "-o", str(exe),
              f"-L{LIB_DIR}", "-lw8a8", "-Wl,-rpath,$ORIGIN/../lib", f"-Wl,-rpath,{LIB_DIR}"],
             verbose)
        return exe

    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, os.cpu_count() or 4)) as ex:
        return list(ex.map(one, srcs))


# CLIs also built with the CPU-verify switch on, into bin/debug/, so that the
# GPU tests can run a debug build without compiling on the GPU box
DEBUG_APPS = ("rocwmma_smoothquant", "rocwmma_gemm_quantized")


def build_debug_apps(verbose: bool = False) -> list[Path]:
    return [exe for name in DEBUG_APPS
            for exe in build_apps(debug=True, verbose=verbose, only=name,
                                  bin_dir=BIN_DIR / "debug")]


def clean() -> None:
    for d in (OBJ_DIR, LIB_DIR, BIN_DIR):
        shutil.rmtree(d, ignore_errors=True)


def main(argv: list[str] | None = None) -> int:
    """Command line; the option letters are the reference build script's
    (build.sh:8-17: -g -t -j -b -i -c -d -v), mapped onto this build."""
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("-g", "--gpu-targets", default=ARCH,
                    help="GPU targets; only gfx950 is built (the kernels are CDNA4 code)")
    ap.add_argument("-t", "--target", default="all_samples",
                    help="all_samples (library + every CLI), w8a8 (library only), or one CLI name")
    ap.add_argument("-j", "--jobs", type=int, default=None, help="parallel compile jobs")
    ap.add_argument("-b", "--build-dir", default=None,
                    help="directory for the CLI executables (default: the package's bin/)")
    ap.add_argument("-i", "--include-dir", default=None,
                    help="accepted for the reference's command line; unused (no rocWMMA headers)")
    ap.add_argument("-c", "--clean", action="store_true", help="remove previous build outputs first")
    ap.add_argument("-d", "--debug", action="store_true",
                    help="CLIs with the CPU-verify switch on (the reference's Debug build)")
    ap.add_argument("--no-apps", action="store_true", help="library only (same as -t w8a8)")
    ap.add_argument("--apps-only", action="store_true",
                    help="CLIs only, linked against the library already built in lib/")
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args(argv)
    targets = [t for t in args.gpu_targets.replace(",", ";").split(";") if t]
    if targets != [ARCH]:
        print(f"[ERROR] GPU targets {args.gpu_targets!r}: this build targets {ARCH} (MI355X) only",
              file=sys.stderr)
        return 1
    if args.clean:
        clean()
    if args.apps_only:
        if not LIB_PATH.exists():
            print(f"[ERROR] --apps-only needs {LIB_PATH} (build the library first)",
                  file=sys.stderr)
            return 1
    else:
        lib = build_library(verbose=args.verbose, jobs=args.jobs)
        print(f"built {lib}")
    if args.no_apps or args.target == "w8a8":
        return 0
    only = None if args.target == "all_samples" else args.target
    for exe in build_apps(debug=args.debug, verbose=args.verbose, only=only,
                          bin_dir=Path(args.build_dir) if args.build_dir else None,
                          jobs=args.jobs):
        print(f"built {exe}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
