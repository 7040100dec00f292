#!/bin/bash
# The rocprofv3 runs behind profiles/: a kernel trace of every benchmark workload
# named below, SQ counter passes and HBM traffic (FETCH_SIZE, WRITE_SIZE) for the
# headline kernels.  Run from the repository root on a GPU host:
#     bash laguna-raw-halo-strix_amd/profile_runs.sh OUTDIR [traces|counters|traffic|all]
# (TRACES="w1 w2 ..." in the environment replaces the list of traced workloads.)
# Raw profiler output and the text summaries go to OUTDIR (the summaries as
# OUTDIR/summaries/*.txt, to be copied into profiles/).  Each profiler run has its
# own time limit; the script stops at the first run that fails.
set -u
OUT=$(realpath -m "${1:-gpurun_out/prof}")
WHAT=${2:-all}
REPO=$(pwd)
SUM="$OUT/summaries"
mkdir -p "$SUM"
cd /tmp && export TMPDIR=/tmp
PS="python3 $REPO/laguna-raw-halo-strix_amd/prof_summary.py"
BENCH="python3 $REPO/bench.py"

run() {  # run NAME ARGS...: one rocprofv3 invocation, stop on failure
    local name=$1
    shift
    echo "== $name: rocprofv3 $*" | sed "s|$REPO|\$REPO|g"
    timeout -k 10 300 rocprofv3 "$@" > "$OUT/$name.log" 2>&1
    local rc=$?
    if [ $rc -ne 0 ]; then
        echo "rocprofv3 run $name ended with status $rc"
        tail -5 "$OUT/$name.log"
        exit $rc
    fi
}

if [ "$WHAT" = all ] || [ "$WHAT" = traces ]; then
    for W in ${TRACES:-q4k_m1 q8_0_m1 q4k_down_silu q4k_m1_k14336 q4k_m1_k20480 q4k_lm_head_m1 q4k_m16_f32 q8_0_m16_f32 \
             q4k_m16_f32_tiled q8_0_m16_f32_tiled q4k_lm_head_m16 lm_head_verify_m16 dflash_block_eager target_token ceil_read_33.1MB \
             ceil_read_17.8MB ceil_empty}; do
        ARGS=(--kernel-trace --stats --output-format csv -d "$OUT/tr_$W" -o run -- $BENCH --workload $W --no-extra --no-cpu)
        run "tr_$W" "${ARGS[@]}"
        $PS trace --dir "$OUT/tr_$W" --out "$SUM/kernel_trace_$W.txt" \
            --cmd "cd /tmp && rocprofv3 --kernel-trace --stats --output-format csv -d OUT -o run -- python3 \$REPO/bench.py --workload $W --no-extra --no-cpu (laguna-raw-halo-strix_amd/profile_runs.sh)"
    done
fi

# workload, kernel name, weights per launch
COUNTED="q4k_m1:k_q4k_m1_dig:58720256 q8_0_m1:k_q80_m1_dig:16777216 q4k_m16_f32_tiled:k_q4k_mm:58720256 q4k_down_silu:k_q4k_m1_wide:58720256"
if [ "$WHAT" = all ] || [ "$WHAT" = counters ]; then
    for E in $COUNTED; do
        IFS=: read -r W K NW <<< "$E"
        run "pmcA_$W" --pmc SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS SQ_INSTS_VMEM SQ_INSTS_SALU SQ_WAVES \
            SQ_BUSY_CYCLES SQ_WAVE_CYCLES GRBM_GUI_ACTIVE --output-format csv -d "$OUT/pmcA_$W" -o run -- \
            $BENCH --pmc --workload $W --steps 20
        run "pmcB_$W" --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_ACTIVE_INST_VALU SQ_LDS_BANK_CONFLICT SQ_WAIT_INST_ANY \
            --output-format csv -d "$OUT/pmcB_$W" -o run -- $BENCH --pmc --workload $W --steps 20
        $PS counters --dirs "$OUT/pmcA_$W" "$OUT/pmcB_$W" --kernel "$K" --weights "$NW" --out "$SUM/counters_$W.txt" \
            --cmd "cd /tmp && rocprofv3 --pmc SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS SQ_INSTS_VMEM SQ_INSTS_SALU SQ_WAVES SQ_BUSY_CYCLES SQ_WAVE_CYCLES GRBM_GUI_ACTIVE --output-format csv -d OUT -o run -- python3 \$REPO/bench.py --pmc --workload $W --steps 20; the same with --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_ACTIVE_INST_VALU SQ_LDS_BANK_CONFLICT SQ_WAIT_INST_ANY (laguna-raw-halo-strix_amd/profile_runs.sh)"
    done
fi

TRAFFIC="q4k_m1:k_q4k_m1_dig q8_0_m1:k_q80_m1_dig q4k_down_silu:k_q4k_m1_wide q4k_m16_f32_tiled:k_q4k_mm"
if [ "$WHAT" = all ] || [ "$WHAT" = traffic ]; then
    for E in $TRAFFIC; do
        IFS=: read -r W K <<< "$E"
        run "pmcf_$W" --pmc FETCH_SIZE --output-format csv -d "$OUT/pmcf_$W" -o run -- $BENCH --pmc --workload $W --steps 20
        run "pmcw_$W" --pmc WRITE_SIZE --output-format csv -d "$OUT/pmcw_$W" -o run -- $BENCH --pmc --workload $W --steps 20
        $PS traffic --fetch "$OUT/pmcf_$W" --write "$OUT/pmcw_$W" --kernel "$K" --out "$SUM/traffic_$W.txt" \
            --cmd "cd /tmp && rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT -o run -- python3 \$REPO/bench.py --pmc --workload $W --steps 20; the WRITE_SIZE run is the same with --pmc WRITE_SIZE (laguna-raw-halo-strix_amd/profile_runs.sh)"
    done
fi
echo "profile_runs: done ($WHAT)"
