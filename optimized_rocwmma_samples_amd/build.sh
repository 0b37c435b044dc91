#!/usr/bin/env bash
# build.sh -- build libw8a8.so and the sample CLIs for MI355X (gfx950).
#
# Options (the letters of the reference's build script):
#   -g, --gpu-targets  GPU targets (only gfx950 is built)
#   -t, --target       all_samples (default), w8a8 (library only) or one CLI name
#   -j, --jobs         parallel compile jobs
#   -b, --build-dir    directory for the CLI executables (default: bin/ beside this script)
#   -i, --include-dir  accepted, unused (no rocWMMA headers are needed)
#   -c, --clean        remove previous build outputs first
#   -d, --debug        CLIs with the CPU-verify switch on
#   --apps-only        CLIs only, against the library already in lib/
#   -v, --verbose      print every compiler command
#   -h, --help         this help
set -euo pipefail
here="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
python3 "${here}/build.py" "$@"
