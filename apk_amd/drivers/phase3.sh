#!/usr/bin/env bash
# Tile-boundary yield: the float64 gate, polling overhead (ABAB), and latency
# with the flag set on the device and by the host (the reference's
# scripts/phase3.sh).
# Usage: apk_amd/drivers/phase3.sh [EVENTS] [extra yield flags...]
source "$(dirname "$0")/common.sh"
EVENTS=${1:-10000}; shift || true
banner "verify"
"$BIN/yield" --mode verify --tasks 20000 "$@"
banner "overhead"
"$BIN/yield" --mode overhead --tasks 200000 --reps 20 --csv "$RAW/phase3_overhead.csv" "$@"
for SET in dev host; do
  banner "latency, $SET-set"
  "$BIN/yield" --mode latency --set "$SET" --events "$EVENTS" --csv "$RAW/phase3_lat_${SET}.csv" "$@"
done
