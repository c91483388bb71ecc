// k_visibility.hip -- flag-notification microbenchmark (counterpart of
// visibility_poll, reference src/yield.cu:216-293): how long a device-scope
// generation store takes to be observed by every polling block, with the
// tile work removed, optionally with DRAM traffic in flight; plus the round
// trip of the polled load itself, per block.
#include "capi.hpp"
#include "device.hpp"

namespace apk {

template <bool LOADED>
__global__ void __launch_bounds__(256) k_visibility(const apk_vis_params P) {
  extern __shared__ float pad[];  // residency parity with a tile kernel
  __shared__ int s_flag;
  const int tid = threadIdx.x, bid = blockIdx.x, G = gridDim.x;
  const int copies = P.flag_copies > 0 ? P.flag_copies : 1;
  const int* myflag = (const int*)((const char*)P.flag + (size_t)(bid % copies) * APK_FLAG_STRIDE);
  const bool isSetter = bid == 0 && P.sched != nullptr;
  if (tid == 0) s_flag = 0;
  if (tid == 0 && P.block_domain)
    P.block_domain[bid] = (int)(xcc_id() * APK_SES_PER_XCD + se_id());
  pad[tid] = (float)tid;
  __syncthreads();
  int lastSeen = 0, nextEv = 0;
  int64_t gBase = 0, it = 0, ldSum = 0, ldMax = 0;
  float acc = 1.0f;
  const size_t gtid = (size_t)bid * 256 + tid;
  const int64_t start = wall_ticks();
  for (;;) {
    for (int i = 0; i < P.work_iters; ++i) acc = fmaf(acc, 1.0000001f, 1e-7f);
    if (LOADED) {
      const float4 v = ((const float4*)P.traffic)[(gtid + (size_t)it * 131071u) %
                                                  (unsigned)P.traffic_len];
      acc += v.x + v.y + v.z + v.w;
    }
    __syncthreads();
    if (tid == 0) {
      const int64_t t0 = wall_ticks();
      const int f = flag_load(myflag);
      // The clock is read once the loaded value is in a register (the asm
      // consumes it, so the compiler waits for the load first).
      asm volatile("" : : "v"(f));
      const int64_t t1 = wall_ticks();
      ldSum += t1 - t0;
      ldMax = (t1 - t0) > ldMax ? (t1 - t0) : ldMax;
      // hard deadline: the block leaves even if it never sees the stop value
      s_flag = (t1 - start > P.max_ticks) ? -1 : f;
      if (isSetter) {
        const int64_t now = wall_ticks();
        if (gBase == 0) gBase = now;
        auto set_all = [&](int v) {
          for (int c = 0; c < copies; ++c)
            flag_store((int*)((char*)P.flag + (size_t)c * APK_FLAG_STRIDE), v);
        };
        if (nextEv < P.num_events) {
          if (now >= gBase + P.sched[nextEv]) {
            P.set_gt[nextEv] = now;
            set_all(++nextEv);
          }
        } else if (now >= gBase + (P.num_events ? P.sched[P.num_events - 1] : 0) +
                              P.stop_after) {
          set_all(-1);
        }
      }
    }
    __syncthreads();
    int f = uniform(s_flag);  // barrier-protected snapshot
    __syncthreads();
    if (f < 0) break;
    if (f > P.num_events) f = P.num_events;
    if (f > lastSeen) {
      const int64_t g = wall_ticks();
      if (tid == 0)
        for (int e = lastSeen; e < f; ++e) P.obs_gt[(size_t)e * G + bid] = g;
      lastSeen = f;
    }
    ++it;
  }
  if (tid == 0) {
    P.iter_count[bid] = it;
    P.load_ticks[2 * bid] = ldSum;
    P.load_ticks[2 * bid + 1] = ldMax;
  }
  P.sink[gtid] = acc + pad[(tid + 1) % 256];
}

}  // namespace apk

extern "C" int apk_visibility(const apk_vis_params* p, int blocks, int lds_bytes,
                              void* stream) {
  using namespace apk;
  APK_REQUIRE(p && p->flag && p->set_gt && p->obs_gt && p->sink && p->iter_count &&
                  p->load_ticks, "visibility: NULL pointer");
  APK_REQUIRE(p->num_events >= 0 && (p->num_events == 0 || p->sched),
              "visibility: schedule");
  APK_REQUIRE(p->stop_after > 0 && p->max_ticks > 0,
              "visibility: stop_after and max_ticks must be > 0 (self-terminating)");
  APK_REQUIRE(p->flag_copies >= 0 && p->flag_copies <= APK_FLAG_MAX_COPIES,
              "visibility: flag_copies=%d", p->flag_copies);
  APK_REQUIRE(!p->loaded || (p->traffic && p->traffic_len > 0), "visibility: traffic");
  APK_REQUIRE(blocks > 0 && lds_bytes >= 1024 && lds_bytes <= 160 * 1024,
              "visibility: blocks=%d lds=%d", blocks, lds_bytes);
  if (p->loaded) {
    APK_HIP(hipFuncSetAttribute((const void*)k_visibility<true>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes));
    hipLaunchKernelGGL(k_visibility<true>, dim3(blocks), dim3(256), lds_bytes,
                       as_stream(stream), *p);
  } else {
    APK_HIP(hipFuncSetAttribute((const void*)k_visibility<false>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes));
    hipLaunchKernelGGL(k_visibility<false>, dim3(blocks), dim3(256), lds_bytes,
                       as_stream(stream), *p);
  }
  APK_LAUNCHED();
  return APK_OK;
}

extern "C" int apk_visibility_occupancy(int lds_bytes, int* blocks_per_cu) {
  using namespace apk;
  APK_REQUIRE(blocks_per_cu && lds_bytes >= 1024 && lds_bytes <= 160 * 1024,
              "visibility_occupancy: lds=%d", lds_bytes);
  APK_HIP(hipFuncSetAttribute((const void*)k_visibility<true>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes));
  int n = 0;
  APK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_visibility<true>, 256, lds_bytes));
  *blocks_per_cu = n;
  return APK_OK;
}
