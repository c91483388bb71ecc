// mid_common.hpp -- shared driver of the midyield and tcyield binaries: yields
// inside the k loop of a pipelined tile (drain + checkpoint/resume), their
// safety, latency and overhead, on any tile engine.
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
