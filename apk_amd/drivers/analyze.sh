#!/usr/bin/env bash
# The analysis ports over a phase-4 grid and OBS1 dumps in results/raw.
# Usage: apk_amd/drivers/analyze.sh [LATENCY_OBS1] [FLOOR_OBS1] [LOADED_OBS1]
source "$(dirname "$0")/common.sh"
ROOT=$(cd "$(dirname "$0")/../.." && pwd)
export PYTHONPATH="$ROOT${PYTHONPATH:+:$PYTHONPATH}"
python3 -m apk_amd.analysis.spread --raw "$RAW" --blocks 32,64,128,256,512 \
  --out results/summary/spread_scaling.csv
if [ $# -ge 2 ]; then
  python3 -m apk_amd.analysis.maxofn --part "MI355X=$1" --floor "MI355X=$2" \
    --out results/summary/heldout_maxofn.csv
fi
if [ $# -ge 3 ]; then
  python3 -m apk_amd.analysis.visibility --run "MI355X:256:floor=$2" \
    --run "MI355X:256:loaded=$3" --out results/summary/visibility.csv
fi
