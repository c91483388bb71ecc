// tiny_oracle.hpp -- `tcyield --mode tiny`: the exactly-once scheduler oracle
// of cfg5 on tiny tasks (one 16x16x16 bf16 MFMA each), by default 1e8 of them
// under device-raised preemption events. Flags: --tasks (1e8), --tiny-batch
// (task ids per pop, 1), --events (1000), --mean-gap-us (exponential gaps,
// 50), --urgent-tiles (urgent tasks per event, 64), --pa / --pb (operand tile
// pools, 64), --blocks-per-cu (2; 4 worker waves per block), --seed (21).
// Reports tasks/s, the exactly-once counts (the reference's ORACLE: PASS /
// FAIL line and exit code, src/yield.cu:630-666) and whether the device's
// background and urgent checksums equal the host's prediction.
#pragma once

namespace host {
int run_tiny_oracle(int argc, char** argv);
}
