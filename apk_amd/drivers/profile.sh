#!/usr/bin/env bash
# rocprofv3 around one command: the kernel trace with per-kernel stats, then
# each counter set in a run of its own (one --pmc run cannot collect more than
# the hardware's per-block counter limits).
# Usage: apk_amd/drivers/profile.sh OUTDIR -- command args...
set -euo pipefail
OUT=$(mkdir -p "$1" && cd "$1" && pwd); shift
[ "${1:-}" = "--" ] && shift
export TMPDIR=${TMPDIR:-/tmp}
rocprofv3 --kernel-trace --stats -f csv -d "$OUT/trace" -o kt -- "$@"
for SET in "FETCH_SIZE" "WRITE_SIZE" \
           "SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS SQ_INSTS_SALU GRBM_GUI_ACTIVE"; do
  name=${SET%% *}
  timeout -s KILL 300 rocprofv3 --pmc $SET --kernel-trace -f csv -d "$OUT/$name" -o p -- "$@"
done
