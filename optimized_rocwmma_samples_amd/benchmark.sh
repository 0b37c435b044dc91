#!/usr/bin/env bash
# benchmark.sh -- run the W8A8 sample CLIs and collect their result lines.
#
# Options: -b DIR, -o FILE, -s a,b, -g N, --csv, --timeout S, --verify, -h.
# The runner itself is benchmark.py (same directory); see its --help.
set -euo pipefail
here="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
python3 "${here}/benchmark.py" "$@"
