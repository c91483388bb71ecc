// k_oracle.hip -- the exactly-once scheduler oracle on tiny tasks.
//
// The reference proves exactly-once execution by counting every completed
// tile in an oracle instantiation of its persistent kernels (src/yield.cu:
// 570-667, src/midyield.cu:760-791, src/tcyield.cu:815-839), at tens of
// millions of full tiles per run. Here the task is one 16x16x16 bf16 MFMA,
// so 1e8 tasks pass through the queue in well under a second and the queue,
// the preempt protocol and the checkpoint path are what is being counted:
//  * every wave of the grid is an independent worker: no barriers, no LDS;
//    lane 0 pops `batch` task ids from its XCD's counter (stealing from the
//    other XCDs' lists once its own is empty) and broadcasts them;
//  * the generation flag is loaded with every pop; between a task's MFMA
//    and its completion a new generation is acted on: a wave that pops one
//    of the event's urgent tasks saves its accumulator tile to HBM, runs
//    urgent tasks until the mini-queue is empty, restores and completes;
//  * completion counts exec_count[t] and adds the task's fingerprint to a
//    per-wave sum, so a lost, duplicated or corrupted task changes either
//    the counts or the checksum the host predicts.
#include "capi.hpp"
#include "device.hpp"

namespace apk {

typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;
constexpr uint64_t kUrgentSalt = 0xD1B54A32D192ED03ull;

// Wrapping sum of a per-lane u64 over the wave (every lane gets the sum).
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), off, 64);
    v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}

// One tiny task: C = A[ia] . B[ib] on the matrix core. Lane l supplies row
// l % 16 of A and column l % 16 of B (k = 4 (l / 16) .. +3) and receives
// C[4 (l / 16) + j][l % 16], j = 0..3.
__device__ __forceinline__ f32x4 tiny_mfma(const uint16_t* A, const uint16_t* Bt, int ia,
                                           int ib) {
  const int l = lane_id();
  const int off = (l & 15) * 16 + 4 * (l >> 4);
  const s16x4 a = *(const s16x4*)(A + (size_t)ia * 256 + off);
  const s16x4 b = *(const s16x4*)(Bt + (size_t)ib * 256 + off);
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, z, 0, 0, 0);
}

// v = wrapping sum over lanes l and registers j of mix64(bits + ((4l+j) << 32)).
__device__ __forceinline__ uint64_t tile_value(const f32x4& c) {
  const uint64_t l4 = (uint64_t)(lane_id() * 4);
  uint64_t h = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    h += mix64((uint64_t)__float_as_uint(c[j]) + ((l4 + j) << 32));
  return wave_sum_u64(h);
}

__global__ void __launch_bounds__(256) k_tiny_oracle(const apk_tiny_params P) {
  const int lane = lane_id();
  const int wave = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  const int home = (int)xcc_id();
  const unsigned N = P.num_tasks;
  const unsigned batch = (unsigned)P.batch;
  const int U = P.urgent_per_event;
  float* slot = P.ckpt + (size_t)wave * 256 + lane * 4;
  const bool setter = P.sched != nullptr && P.num_events > 0 && wave == 0;

  uint64_t sumBg = 0, sumU = 0, yields = 0, urgentRun = 0;
  int lastSeen = 0, nextEv = 0;
  int64_t base = 0;
  int q = 0;  // lists visited: own XCD's first, then the others in turn

  // Serve every event raised since the last look: log nothing, pop urgent
  // tasks; on the first pop save `c` (the in-flight tile) and restore it at
  // the end. Returns the tile unchanged in value.
  auto serve = [&](int f, f32x4& c, bool live) {
    if (f > P.num_events) f = P.num_events;
    for (int e = lastSeen; e < f; ++e) {
      bool saved = false;
      for (;;) {
        int u = 0;
        if (lane == 0) u = fetch_add_i32(&P.uq_next[e], 1);
        u = __builtin_amdgcn_readfirstlane(u);
        if (u >= U) break;
        if (live && !saved) {  // yield: the in-flight tile goes to HBM
          *(f32x4*)slot = c;
          saved = true;
          ++yields;
        }
        const uint64_t id = (uint64_t)e * (uint64_t)U + (uint64_t)u;
        const f32x4 cu = tiny_mfma(P.A, P.Bt, (int)((id * 7 + 3) % (uint64_t)P.pa),
                                   (int)((id * 13 + 5) % (uint64_t)P.pb));
        const uint64_t v = tile_value(cu);
        sumU += mix64(v + id * kGolden + kUrgentSalt);
        ++urgentRun;
        if (lane == 0) fetch_add_i32(&P.u_exec_count[e], 1);
      }
      if (saved) c = *(const volatile f32x4*)slot;  // restore
    }
    if (f > lastSeen) lastSeen = f;
  };

  for (;;) {
    // The setter raises the events that are due (device clock).
    if (setter && lane == 0) {
      const int64_t now = wall_ticks();
      if (base == 0) base = now;
      if (nextEv < P.num_events && now >= base + P.sched[nextEv]) {
        P.set_gt[nextEv] = now;
        flag_store(P.flag, ++nextEv);
      }
    }
    // Pop a batch: lane 0 does the atomic, the wave reads lane 0's result.
    unsigned first = 0xffffffffu, count = 0;
    while (q < APK_QUEUE_XCDS) {
      const int l = (home + q) & (APK_QUEUE_XCDS - 1);
      const unsigned b = (unsigned)(((uint64_t)l * N) / APK_QUEUE_XCDS);
      const unsigned n = (unsigned)(((uint64_t)(l + 1) * N) / APK_QUEUE_XCDS) - b;
      unsigned j = 0xffffffffu;
      if (lane == 0 && n > 0) j = fetch_add_u32(&P.next_task[l], batch);
      j = (unsigned)__builtin_amdgcn_readfirstlane((int)j);
      if (n > 0 && j < n) {
        first = b + j;
        count = min(batch, n - j);
        break;
      }
      ++q;  // this list is exhausted
    }
    int f = 0;
    if (lane == 0) f = flag_load(P.flag);
    f = __builtin_amdgcn_readfirstlane(f);
    if (count == 0) {
      // Last look before leaving: every raised event must be served.
      f32x4 none = {0.f, 0.f, 0.f, 0.f};
      if (f > lastSeen) serve(f, none, false);
      break;
    }
    for (unsigned i = 0; i < count; ++i) {
      const unsigned t = first + i;
      f32x4 c = tiny_mfma(P.A, P.Bt, (int)(t % (unsigned)P.pa),
                          (int)((t / (unsigned)P.pa) % (unsigned)P.pb));
      if (i == 0 && f > lastSeen) serve(f, c, true);  // preempt between MFMA and completion
      if (P.c_debug && t < P.n_debug) *(f32x4*)(P.c_debug + (size_t)t * 256 + lane * 4) = c;
      const uint64_t v = tile_value(c);
      sumBg += mix64(v + (uint64_t)t * kGolden);
      if (lane == 0) fetch_add_i32(&P.exec_count[t], 1);
    }
  }
  if (lane == 0) {
    __hip_atomic_fetch_add(&P.checksum[0], (unsigned long long)sumBg, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_fetch_add(&P.checksum[1], (unsigned long long)sumU, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    if (P.stats) {
      __hip_atomic_fetch_add(&P.stats[0], (unsigned long long)yields, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_add(&P.stats[1], (unsigned long long)urgentRun, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace apk

extern "C" int apk_tiny_oracle(const apk_tiny_params* p, int blocks, void* stream) {
  using namespace apk;
  APK_REQUIRE(p != nullptr, "tiny_oracle: params is NULL");
  APK_REQUIRE(p->next_task && p->A && p->Bt && p->exec_count && p->checksum && p->flag &&
                  p->ckpt,
              "tiny_oracle: NULL pointer");
  APK_REQUIRE(p->batch >= 1 && p->pa >= 1 && p->pb >= 1, "tiny_oracle: batch=%d pa=%d pb=%d",
              p->batch, p->pa, p->pb);
  APK_REQUIRE(blocks > 0, "tiny_oracle: blocks=%d", blocks);
  APK_REQUIRE(p->num_events >= 0 && p->urgent_per_event >= 0,
              "tiny_oracle: num_events=%d urgent_per_event=%d", p->num_events,
              p->urgent_per_event);
  if (p->num_events > 0)
    APK_REQUIRE(p->sched && p->set_gt && p->uq_next && p->u_exec_count,
                "tiny_oracle: events need sched, set_gt, uq_next and u_exec_count");
  APK_REQUIRE(!p->c_debug || p->n_debug <= p->num_tasks, "tiny_oracle: n_debug=%u",
              p->n_debug);
  hipLaunchKernelGGL(k_tiny_oracle, dim3(blocks), dim3(256), 0, as_stream(stream), *p);
  APK_LAUNCHED();
  return APK_OK;
}
