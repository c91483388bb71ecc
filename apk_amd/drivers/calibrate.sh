#!/usr/bin/env bash
# Tile calibration sweep over the per-tile K (the reference's scripts/calibrate.sh:
# K = 32..512, default 48x48 tiles, verification on). The device wall clock is
# 100 MHz and needs no lock, so the clock argument only feeds --sm-clock-mhz.
# Usage: apk_amd/drivers/calibrate.sh [SM_MHZ] [extra persistent flags...]
source "$(dirname "$0")/common.sh"
SM_MHZ=${1:-0}; shift || true
for K in 32 64 128 256 512; do
  banner "K=$K"
  "$BIN/persistent" --k "$K" --sm-clock-mhz "$SM_MHZ" --csv "$RAW/calib_k${K}.csv" "$@"
done
