// midyield -- the reference's bin/midyield (src/midyield.cu:348-793): yields
// inside the k loop of a pipelined tile. The driver, its flags and its
// semantics are in mid_common.hpp; this binary's defaults are the
// reference's (64x64 fp32 VALU tile, --k 64, 48x48 tiles, 200,000 tasks).
#include "mid_common.hpp"

int main(int argc, char** argv) {
  const host::MidVariant v{"midyield", "valu64", 64, 48, 200000, false};
  return host::run_midyield(argc, argv, v);
}
