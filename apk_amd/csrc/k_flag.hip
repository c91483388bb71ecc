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

}  // namespace apk

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
