#!/usr/bin/env bash
# The latency / overhead surface over resident blocks x poll period (the
# reference's scripts/phase4.sh), with MI355X block counts: 32 .. 512 (up to two
# 64x64 VALU blocks on each of the 256 CUs). analyze.sh summarises the result.
# Usage: apk_amd/drivers/phase4.sh [EVENTS] [BLOCKS...]
source "$(dirname "$0")/common.sh"
EVENTS=${1:-10000}; shift || true
BLOCKS=${*:-32 64 128 256 512}
for B in $BLOCKS; do
  for P in 1 2 4 8; do
    banner "blocks=$B poll-every=$P: latency"
    "$BIN/yield" --mode latency --set dev --events "$EVENTS" --blocks "$B" --poll-every "$P" \
      --csv "$RAW/phase4_lat_b${B}_p${P}.csv"
    banner "blocks=$B poll-every=$P: overhead"
    "$BIN/yield" --mode overhead --tasks $((B * 700)) --reps 20 --blocks "$B" --poll-every "$P" \
      --csv "$RAW/phase4_ovh_b${B}_p${P}.csv"
  done
done
