// tcyield -- preemptible bf16 GEMM on the gfx950 matrix cores: safety,
// latency, overhead and tile calibration of k-stage and chunk yields.
//
// Measurement surface of the reference's bin/tcyield (src/tcyield.cu:
// 384-842): flags --mode events|verify|overhead|calibrate --discipline
// drain|naive|poison --poll off|pe|stage|issue --k 256 --tiles-m 8
// --tiles-n 8 --events 10000 --tasks 20000 --reps 20 --gap-min-us 150
// --gap-max-us 400 --blocks 0 --warmup-events 100 --oracle 0 --csv, and the
// per-event CSV "event,lat_us,lat_excl_setter_us,first_us,claimer,e2e_us,
// bad_elems,site,complete".
//
// The reference's 128x128 fp16 wmma tile becomes the BF16X256 engine:
// 256x256 tiles of bf16 operands with fp32 accumulation on
// v_mfma_f32_32x32x16_bf16 (B held transposed on the device); --engine
// bf16x128 selects the one-wave 128x128 bf16 tile built for 4 blocks per CU
// (--blocks 1024), bf16x256x128 the four-wave 256x128 tile built for 2 blocks
// per CU (--blocks 512). Inputs are normal(0,1) rounded to bf16; the float64
// reference multiplies the bf16-quantized values (src/tcyield.cu:459-473).
// --poll pe is the chunk (tile-boundary) poll, --poll issue the
// window-forcing issue site (checkpoint before any wait). Every other flag and
// addition is the midyield driver's: --engine, --gemm-k, --resume,
// --urgent-m/-n/-k, --arrival, --mean-gap-us, --seed, --flag-copies,
// --verify-rows.
// --mode tiny runs the scheduler oracle on 1e8 tiny tasks (tiny_oracle.hpp).
#include "mid_common.hpp"
#include "tiny_oracle.hpp"
#include "host_common.hpp"

#include <cstring>
#include <string>
#include <vector>

int main(int argc, char** argv) {
  if (std::strcmp(host::parse_str(argc, argv, "--mode", "events"), "tiny") == 0)
    return host::run_tiny_oracle(argc, argv);
  // --poll pe (the reference's tile-boundary poll) is midyield's "boundary".
  std::vector<char*> args(argv, argv + argc);
  static char boundary[] = "boundary";
  for (int i = 1; i + 1 < argc; ++i)
    if (std::strcmp(args[i], "--poll") == 0 && std::strcmp(args[i + 1], "pe") == 0)
      args[i + 1] = boundary;
  const host::MidVariant v{"tcyield", "bf16x256", 256, 8, 20000, true};
  return host::run_midyield(argc, args.data(), v);
}
