#!/usr/bin/env bash
# Mid-pipeline yield safety (the reference's scripts/phase5.sh): drain and
# poison gates, events per discipline at the stage site, the boundary-poll
# comparator, overhead per poll site. Add `--poll issue` runs for the
# window-forcing site.
# Usage: apk_amd/drivers/phase5.sh [EVENTS] [extra midyield flags...]
source "$(dirname "$0")/common.sh"
EVENTS=${1:-10000}; shift || true
for D in drain poison; do
  banner "verify: $D"
  "$BIN/midyield" --mode verify --discipline "$D" --tasks 20000 "$@"
done
for D in drain naive poison; do
  banner "events: $D, stage poll"
  "$BIN/midyield" --mode events --discipline "$D" --events "$EVENTS" --csv "$RAW/phase5_${D}.csv" "$@"
done
banner "events: drain, boundary poll"
"$BIN/midyield" --mode events --discipline drain --poll boundary --events "$EVENTS" \
  --csv "$RAW/phase5_drain_boundary.csv" "$@"
for P in stage boundary; do
  banner "overhead: poll=$P"
  "$BIN/midyield" --mode overhead --poll "$P" --tasks 200000 --reps 20 "$@"
done
