// mid_common.hpp -- shared driver of the midyield and tcyield binaries: yields
// inside the k loop of a pipelined tile (drain + checkpoint/resume), their
// safety, latency and overhead, on any tile engine.
//
// Measurement surface of the reference's bin/midyield (src/midyield.cu:
// 348-793): flags --mode events|verify|overhead --discipline drain|naive|
// poison --poll off|boundary|stage|issue --k 64 --tiles-m 48 --tiles-n 48
// --events 10000 --tasks 200000 --reps 20 --gap-min-us 150 --gap-max-us 400
// --blocks 0 --warmup-events 100 --oracle 0 --csv, the SAFETY / latency /
// oracle summary lines and the per-event CSV "event,lat_us,
// lat_excl_setter_us,first_us,claimer,e2e_us,cu_max_rel,corrupt,complete,
// site" (extra columns appended).
//
// MI355X semantics. The tile walks K in LDS k-stages of a 3-slot ring fed by
// direct-to-LDS loads; a stage poll sits before every stage, where stage s is
// resident and stage s+1 may still be in flight. A yielding block drains
// (vmcnt 0) -- unless --discipline naive -- checkpoints its accumulators and
// the two live stages to HBM (--resume ckpt; acc = accumulators only and
// re-fetch; restart = the reference's abandon-and-restart), runs the event's
// urgent tiles through the same ring, restores and continues. Safety is
// checked three ways: every event's urgent output (one per event, the
// reference's CuAll) against float64 and bit for bit against the
// non-preemptible urgent GEMM; every background task's fingerprint against
// the same tile computed without preemption; and C against float64.
// --discipline poison adds +1.0 to one staged B value of every urgent tile,
// so every claimed event must be flagged corrupt (src/midyield.cu:146-147).
// --poll issue is the window-forcing issue site (src/midyield.cu:246-258):
// the next stages' loads go out, the flag is polled right behind them and a
// yield checkpoints before any wait, so --discipline naive can save a stage
// still in flight.
// Additions: --engine valu64|mfma128|bf16x256|bf16x128|bf16x256x128 (default valu64;
// --dtype fp32|bf16 picks the default or bf16x256),
// --dump-obs PATH (the OBS1 observation matrix), --gemm-k K (depth of
// the background GEMM, default --k), --resume ckpt|acc|restart, --urgent-m/
// -n/-k (default one tile of depth --k), --arrival uniform|exp,
// --mean-gap-us, --seed, --flag-copies, --verify-rows (float64 rows of C),
// --poll-every N (--poll boundary: a site at every N-th k-chunk boundary,
// counted across tasks), --prewarm-ms T (--mode calibrate: T ms of untimed
// runs before the timed one), --fingerprints 0|1 (default 1: fingerprint
// every background task against its unpreempted tile; 0 for latency runs,
// since hashing a tile holds its block off its poll sites).
#pragma once

namespace host {

struct MidVariant {
  const char* name;        // binary name in messages
  const char* engine;      // default --engine
  int k;                   // default --k (per-tile K chunk)
  int tiles;               // default --tiles-m / --tiles-n
  unsigned tasks;          // default --tasks
  bool tcCsv;              // per-event CSV in the tcyield column order
};

int run_midyield(int argc, char** argv, const MidVariant& v);

}  // namespace host
