#!/usr/bin/env bash
# Reserved capacity against the cooperative hand-off over urgent sizes (the
# reference's scripts/pareto.sh). On MI355X a reservation needs one free slot
# in every (XCD, shader engine) domain, so R runs past 32.
# Usage: apk_amd/drivers/pareto.sh [TRIALS] [EVENTS]
source "$(dirname "$0")/common.sh"
TRIALS=${1:-10000}
EVENTS=${2:-10000}
mkdir -p "$RAW/pareto"
for R in 1 2 4 8 16 32 64; do
  for U in 1 4 16; do
    "$BIN/urgent_baseline" --mode sat --reserve "$R" --urgent-blocks "$U" --trials "$TRIALS" \
      --csv "$RAW/pareto/res_R${R}_U${U}.csv"
  done
done
"$BIN/urgent_baseline" --mode sat --urgent-blocks 1 --trials 2000 --csv "$RAW/pareto/res_R0_U1.csv"
for U in 1 4 16; do
  "$BIN/yield" --mode latency --set dev --events "$EVENTS" --urgent-tiles "$U" \
    --csv "$RAW/pareto/coop_U${U}.csv"
done
"$BIN/yield" --mode overhead --tasks 200000 --reps 20 --csv "$RAW/pareto/coop_ovh.csv"
