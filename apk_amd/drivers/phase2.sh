#!/usr/bin/env bash
# Urgent-task wait with no yielding, at the three occupancy shapes (the
# reference's scripts/phase2.sh).
# Usage: apk_amd/drivers/phase2.sh [TRIALS] [extra urgent_baseline flags...]
source "$(dirname "$0")/common.sh"
TRIALS=${1:-500}; shift || true
for MODE in sat sat-1 1persm; do
  banner "mode=$MODE"
  "$BIN/urgent_baseline" --mode "$MODE" --trials "$TRIALS" --csv "$RAW/phase2_${MODE}.csv" "$@"
done
