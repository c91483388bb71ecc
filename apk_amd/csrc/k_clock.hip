// k_clock.hip -- the engine clock under load, read on the device.
//
// The reference locks the clock and reads it back under load with
// nvidia-smi (scripts/lock_clocks.sh:15-25). On MI355X the engine clock moves
// with power from dispatch to dispatch, so each throughput figure here is
// reported beside the clock it ran at: one wave per probe block sits beside
// the running kernel (no LDS, a few registers, so it is dispatched next to a
// fully resident grid) and counts shader-clock cycles (s_memtime) against the
// constant-rate wall clock (s_memrealtime) over a window; cycles / ticks x
// the wall-clock rate = the mean engine clock of its CU over that window.
#include "capi.hpp"
#include "device.hpp"

namespace apk {

__global__ void __launch_bounds__(64) k_clock_probe(long long* out, long long window) {
  if (threadIdx.x != 0) return;
  const int64_t w0 = wall_ticks();
  const int64_t c0 = (int64_t)__builtin_amdgcn_s_memtime();
  int64_t w1 = w0;
  while (w1 - w0 < window) {
    __builtin_amdgcn_s_sleep(64);
    w1 = wall_ticks();
  }
  const int64_t c1 = (int64_t)__builtin_amdgcn_s_memtime();
  long long* o = out + 4 * (size_t)blockIdx.x;
  o[0] = c1 - c0;
  o[1] = w1 - w0;
  o[2] = (long long)xcc_id();
  o[3] = w0;
}

}  // namespace apk

extern "C" int apk_clock_probe(long long* out, int blocks, long long window_ticks,
                               void* stream) {
  using namespace apk;
  APK_REQUIRE(out != nullptr, "clock_probe: out is NULL");
  APK_REQUIRE(blocks > 0 && blocks <= 1024, "clock_probe: blocks=%d (1..1024)", blocks);
  APK_REQUIRE(window_ticks > 0 && window_ticks <= 6000000000LL,
              "clock_probe: window_ticks=%lld (1 tick .. 60 s)", window_ticks);
  hipLaunchKernelGGL(k_clock_probe, dim3(blocks), dim3(64), 0, as_stream(stream), out,
                     window_ticks);
  APK_LAUNCHED();
  return APK_OK;
}
