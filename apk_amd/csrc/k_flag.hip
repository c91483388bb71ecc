// k_flag.hip -- raising the generation flag from a stream.
//
// The reference raises events from the host with a cudaMemcpyAsync of the
// flag on a control stream (src/yield.cu:845-858), or from block 0 of the
// persistent kernel itself (src/yield.cu:186-195). For the retreat arm the
// signal must travel with the urgent work on the urgent stream: one wave,
// no LDS and a handful of registers, so the dispatcher places it beside a
// fully resident persistent grid the moment the stream reaches it.
#include "capi.hpp"
#include "device.hpp"

namespace apk {

__global__ void __launch_bounds__(64) k_raise_flag(int* flag, int copies, int value,
                                                   long long* set_gt) {
  if (threadIdx.x != 0) return;
  const int64_t now = wall_ticks();
  for (int c = 0; c < copies; ++c)
    flag_store((int*)((char*)flag + (size_t)c * APK_FLAG_STRIDE), value);
  if (set_gt) *set_gt = now;
}

// Calibration probe of the host-set mode: the device tick at which a flag
// written by the host is first read back non-zero. Bounded by max_ticks.
__global__ void __launch_bounds__(64) k_spin_flag(const int* flag, int system_scope,
                                                  long long max_ticks, long long* out) {
  if (threadIdx.x != 0) return;
  const int64_t t0 = wall_ticks();
  for (;;) {
    const int v = system_scope
                      ? __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM)
                      : flag_load(flag);
    const int64_t now = wall_ticks();
    if (v != 0) {
      out[0] = now;
      out[1] = v;
      return;
    }
    if (now - t0 > max_ticks) {
      out[0] = -1;
      out[1] = 0;
      return;
    }
  }
}

}  // namespace apk

extern "C" int apk_spin_flag(const int* flag, int system_scope, long long max_ticks,
                             long long* out, void* stream) {
  using namespace apk;
  APK_REQUIRE(flag != nullptr && out != nullptr, "spin_flag: NULL pointer");
  APK_REQUIRE(max_ticks > 0, "spin_flag: max_ticks=%lld must be > 0", max_ticks);
  hipLaunchKernelGGL(k_spin_flag, dim3(1), dim3(64), 0, as_stream(stream), flag,
                     system_scope ? 1 : 0, max_ticks, out);
  APK_LAUNCHED();
  return APK_OK;
}

extern "C" int apk_raise_flag(int* flag, int flag_copies, int value, long long* set_gt,
                              void* stream) {
  using namespace apk;
  APK_REQUIRE(flag != nullptr, "raise_flag: flag is NULL");
  APK_REQUIRE(flag_copies >= 1 && flag_copies <= APK_FLAG_MAX_COPIES,
              "raise_flag: flag_copies=%d", flag_copies);
  hipLaunchKernelGGL(k_raise_flag, dim3(1), dim3(64), 0, as_stream(stream), flag, flag_copies,
                     value, set_gt);
  APK_LAUNCHED();
  return APK_OK;
}
