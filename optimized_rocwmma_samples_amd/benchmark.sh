#!/usr/bin/env bash
# =============================================================================
# benchmark.sh -- run the W8A8 path's sample CLIs and collect their results
#
# Same options, report and CSV as the reference's benchmark.sh (options
# :5-15, result extraction :178-189), over the binaries this package builds
# (`python -m optimized_rocwmma_samples_amd.build`).  The CSV gains a %peak
# column: GB/s against 8 TB/s HBM3E, TFlops/s against 5.0 POP/s dense int8.
#
# Usage:
#   ./benchmark.sh [OPTIONS]
#
# Options:
#   -b, --build-dir   Directory of the CLIs (default: <package>/bin)
#   -o, --output      Output report file (default: ./benchmark_results.txt)
#   -s, --samples     Comma-separated sample names to run (default: all)
#   -g, --gpu         GPU device index (default: 0)
#   --csv             Also write CSV results (<output>.csv)
#   --timeout         Per-sample timeout in seconds (default: 120)
#   --verify          Run every CLI with its CPU check (--verify)
#   -h, --help        Show this help
# =============================================================================
set -uo pipefail

SCRIPT_DIR="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
BUILD_DIR="${SCRIPT_DIR}/bin"
OUTPUT_FILE="$(pwd)/benchmark_results.txt"
SAMPLES_FILTER=""
GPU_INDEX=0
WRITE_CSV=0
TIMEOUT_SEC=120
VERIFY=""

while [[ $# -gt 0 ]]; do
    case "$1" in
        -b|--build-dir)  BUILD_DIR="$2";      shift 2 ;;
        -o|--output)     OUTPUT_FILE="$2";    shift 2 ;;
        -s|--samples)    SAMPLES_FILTER="$2"; shift 2 ;;
        -g|--gpu)        GPU_INDEX="$2";      shift 2 ;;
        --csv)           WRITE_CSV=1;         shift ;;
        --timeout)       TIMEOUT_SEC="$2";    shift 2 ;;
        --verify)        VERIFY="--verify";   shift ;;
        -h|--help)       sed -n '2,24p' "$0" | sed 's/^# \?//'; exit 0 ;;
        *) echo "[ERROR] Unknown option: $1"; exit 1 ;;
    esac
done

[[ -d "${BUILD_DIR}" ]] || {
    echo "[ERROR] Build dir not found: ${BUILD_DIR}"
    echo "        Run python -m optimized_rocwmma_samples_amd.build first."
    exit 1
}

export HIP_VISIBLE_DEVICES="${GPU_INDEX}"
CSV_FILE="${OUTPUT_FILE%.txt}.csv"
PEAK_GBPS=8000
PEAK_TFLOPS=5000
TS=$(date '+%Y-%m-%d %H:%M:%S')
ROCM_VER=$(cat /opt/rocm/.info/version 2>/dev/null || echo "unknown")

# "binary|args|description"
declare -a ALL_SAMPLES=(
    "rocwmma_smoothquant|3328 4096|SmoothQuant FP16->INT8 N=4096"
    "rocwmma_smoothquant|3328 8192|SmoothQuant FP16->INT8 N=8192"
    "rocwmma_smoothquant|2048 4096|SmoothQuant config 1 (2048x4096)"
    "rocwmma_moe_smoothquant||MoE SmoothQuant (per-expert scale)"
    "rocwmma_rmsnorm2d|3328 4096|RMSNorm2D + Add+RMSNorm fused (+ SmoothQuant)"
    "rocwmma_gemm_quantized||W8A8 int8 GEMM (per-token x per-channel dequant)"
    "rocwmma_gemm_quantized|--sample-layout|W8A8 int8 GEMM, sample layout + tensor scales"
    "w8a8_fused_sq_gemm||Fused SmoothQuant + GEMM, Llama-3-8B projections"
    "rocwmma_gemm_splitk||Decode GEMM (split-K inside the block)"
    "rocwmma_flatmm||GEMM over packed (pre-shuffled) weights"
    "rocwmma_grouped_gemm||Grouped GEMM (variable-size groups)"
    "rocwmma_topk_softmax||TopK Softmax (wave-per-token)"
    "rocwmma_moe_sorting||MoE Token Sorting (stable counting sort)"
    "rocwmma_fused_moe||MoE FFN (route+sort+quant+GEMM+SiLU*up+GEMM+combine)"
)

if [[ -n "${SAMPLES_FILTER}" ]]; then
    IFS=',' read -ra FILTER_ARR <<< "${SAMPLES_FILTER}"
    declare -a FILTERED=()
    for entry in "${ALL_SAMPLES[@]}"; do
        bin="${entry%%|*}"
        for f in "${FILTER_ARR[@]}"; do
            [[ "${bin}" == *"${f}"* ]] && FILTERED+=("${entry}") && break
        done
    done
    ALL_SAMPLES=("${FILTERED[@]}")
fi
TOTAL=${#ALL_SAMPLES[@]}

HEADER="================================================================================
 W8A8 SmoothQuant path (MI355X gfx950) Benchmark Report
================================================================================
 Date       : ${TS}
 GPU        : device ${GPU_INDEX}
 ROCm       : ${ROCM_VER}
 Build dir  : ${BUILD_DIR}
 Timeout    : ${TIMEOUT_SEC}s per sample
================================================================================"
echo "${HEADER}"
echo "${HEADER}" > "${OUTPUT_FILE}"
[[ "${WRITE_CSV}" -eq 1 ]] && echo "sample,description,metric,value,unit,pct_peak" > "${CSV_FILE}"

pct() { awk -v v="$1" -v p="$2" 'BEGIN{printf "%.1f", 100*v/p}'; }

PASS=0; FAIL=0; SKIP=0
for entry in "${ALL_SAMPLES[@]}"; do
    IFS='|' read -r BIN ARGS DESC <<< "${entry}"
    BINARY="${BUILD_DIR}/${BIN}"
    IDX=$((PASS+FAIL+SKIP+1))
    printf "\n [%2d/%d] %-28s  %s\n" "${IDX}" "${TOTAL}" "${BIN}" "${DESC}"
    printf "\n[%d/%d] %s | %s\n  Args: %s\n" "${IDX}" "${TOTAL}" "${BIN}" "${DESC}" \
        "${ARGS:-<defaults>}" >> "${OUTPUT_FILE}"
    if [[ ! -x "${BINARY}" ]]; then
        echo "  [SKIP] Binary not found: ${BINARY}"
        echo "  [SKIP] Binary not found" >> "${OUTPUT_FILE}"
        ((SKIP++)); continue
    fi
    EXIT_CODE=0
    RESULT=$(timeout -k 10 "${TIMEOUT_SEC}s" "${BINARY}" ${ARGS} ${VERIFY} 2>&1) || EXIT_CODE=$?
    if [[ ${EXIT_CODE} -eq 124 || ${EXIT_CODE} -eq 137 ]]; then
        echo "  [TIMEOUT] Killed after ${TIMEOUT_SEC}s"
        echo "  [TIMEOUT]" >> "${OUTPUT_FILE}"
        ((FAIL++)); continue
    fi
    if [[ ${EXIT_CODE} -ne 0 ]]; then
        echo "  [FAIL] Exit code ${EXIT_CODE}"
        echo "${RESULT}" | tail -3
        printf "  [FAIL] exit=%d\n%s\n" "${EXIT_CODE}" "$(echo "${RESULT}" | tail -3)" >> "${OUTPUT_FILE}"
        ((FAIL++)); continue
    fi
    echo "${RESULT}"
    echo "${RESULT}" >> "${OUTPUT_FILE}"
    ((PASS++))
    if [[ "${WRITE_CSV}" -eq 1 ]]; then
        label="${DESC}"
        while IFS= read -r line; do
            l=$(echo "${line}" | grep -oP '^\[.*?\]' | head -1 | tr -d '[]') || true
            if [[ -n "${l}" ]]; then
                dims=$(echo "${line}" | grep -oP '^\[.*?\]\s*\K[^ ]+=[^ ]+( [^ ]+=[^ ]+)*' | head -1) || true
                label="${l} ${dims}"
            fi
            tf=$(echo "${line}" | grep -oP '[\d.]+(?=\s+TFlops/s)' | head -1) || true
            [[ -n "${tf:-}" ]] && echo "${BIN},\"${DESC}\",\"${label}\",${tf},TFlops/s,$(pct "${tf}" "${PEAK_TFLOPS}")" >> "${CSV_FILE}"
            bw=$(echo "${line}" | grep -oP '[\d.]+(?=\s+GB/s)' | head -1) || true
            [[ -n "${bw:-}" ]] && echo "${BIN},\"${DESC}\",\"${label} bw\",${bw},GB/s,$(pct "${bw}" "${PEAK_GBPS}")" >> "${CSV_FILE}"
        done <<< "${RESULT}"
    fi
done

SUMMARY="
================================================================================
 Benchmark Summary
================================================================================
 Total    : ${TOTAL}
 Passed   : ${PASS}
 Failed   : ${FAIL}
 Skipped  : ${SKIP}
 Output   : ${OUTPUT_FILE}"
[[ "${WRITE_CSV}" -eq 1 ]] && SUMMARY+="
 CSV      : ${CSV_FILE}"
SUMMARY+="
================================================================================"
echo "${SUMMARY}"
echo "${SUMMARY}" >> "${OUTPUT_FILE}"
[[ ${FAIL} -eq 0 ]]
