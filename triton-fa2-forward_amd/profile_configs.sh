#!/bin/bash
# The rocprofv3 runs behind profiles/ (run on the MI355X box from the repository root):
#
#     bash triton-fa2-forward_amd/profile_configs.sh gpurun_out/prof C3 C2 C4 C5
#     python triton-fa2-forward_amd/rocprof_summary.py --root gpurun_out/prof --configs C3 C2 C4 C5
#
# Per config: one kernel trace over bench.py, then one counter run per counter group over
# profile_target.py (three launches and a 1 GiB calibration copy). Counter runs never combine
# --pmc with a tracing option, and each has a time limit of its own; the script stops at the first
# failure. The command lines are the ones rocprof_summary.commands() quotes in the summaries.
set -o pipefail
ROOT_OUT=${1:?output folder}
shift
export TMPDIR=/tmp
mkdir -p "$ROOT_OUT"
SQ="SQ_WAVES SQ_INSTS_MFMA SQ_INSTS_VALU SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_WAVE_CYCLES GRBM_GUI_ACTIVE"
UTIL="SQ_LDS_IDX_ACTIVE SQ_ACTIVE_INST_VALU SQ_VALU_MFMA_COEXEC_CYCLES SQ_INSTS_VALU_TRANS_F32 SQ_INST_CYCLES_SALU SQ_VALU_MFMA_BUSY_CYCLES SQ_WAIT_INST_LDS GRBM_GUI_ACTIVE"
for CFG in "$@"; do
  TARGET="python3 triton-fa2-forward_amd/profile_target.py --config $CFG --launches 3 --copy-mib 1024"
  echo "profile_configs: $CFG trace" 
  timeout -k 10 300 rocprofv3 --kernel-trace --stats --output-format csv -d "$ROOT_OUT/${CFG}_trace" -o trace \
    -- python3 bench.py --config "$CFG" --no-cpu-baseline --flush-iters 0 > "$ROOT_OUT/${CFG}_trace.log" 2>&1 || exit 1
  for PASS in fetch write sq util; do
    case $PASS in
      fetch) CTRS=FETCH_SIZE ;;
      write) CTRS=WRITE_SIZE ;;
      sq) CTRS=$SQ ;;
      util) CTRS=$UTIL ;;
    esac
    echo "profile_configs: $CFG $PASS"
    timeout -s KILL 90 rocprofv3 --pmc $CTRS --output-format csv -d "$ROOT_OUT/${CFG}_${PASS}" -o pmc \
      -- $TARGET > "$ROOT_OUT/${CFG}_${PASS}.log" 2>&1 || exit 1
  done
done
echo "profile_configs: done"
