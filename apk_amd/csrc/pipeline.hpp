// pipeline.hpp -- engine-independent pieces of the persistent kernels:
// the 3-slot direct-to-LDS software pipeline, flag sampling through LDS, the
// bit-exact tile fingerprint, and checkpoint save/restore of accumulators and
// LDS stages.
#pragma once
#include <type_traits>
#include "device.hpp"

#define APK_PROTO_FN __device__ __forceinline__
#include "protocol.hpp"

namespace apk {

// ---------------------------------------------------------------------------
// The scheduler protocol (work queue, resume ring, generations) lives in
// protocol.hpp, shared with the CPU protocol simulator; here it runs on the
// device's agent-scope atomics, fences, wall clock and s_sleep.
struct DevPlat {
  static __device__ __forceinline__ unsigned fetch_add(unsigned* p, unsigned v) {
    return fetch_add_u32(p, v);
  }
  static __device__ __forceinline__ unsigned load(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  static __device__ __forceinline__ int load(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  static __device__ __forceinline__ void store(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // The resume ring's payload (checkpoint slot, entry fields) is written
  // through with agent-coherent stores (CPOL_SC1 / relaxed agent atomics),
  // so publishing it needs only those stores to have completed: no L2
  // write-back, which with every worker retreating at once serialised 32
  // whole-L2 write-backs per XCD.
  static __device__ __forceinline__ void publish_fence() { wait_vmcnt<0>(); }
  static __device__ __forceinline__ void acquire() {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  static __device__ __forceinline__ int64_t ticks() { return wall_ticks(); }
  static __device__ __forceinline__ void pause() { __builtin_amdgcn_s_sleep(8); }
};

using TaskQueue = proto::TaskQueue<DevPlat>;
using proto::RQ_FULL;
using proto::RQ_NONE;
using proto::RQ_STUCK;
// Thread-0 only, each of them.
__device__ __forceinline__ unsigned rq_reserve(unsigned* ctl, unsigned cap, const int* en) {
  return proto::rq_reserve<DevPlat>(ctl, cap, en);
}
__device__ __forceinline__ unsigned rq_pop(unsigned* ctl) { return proto::rq_pop<DevPlat>(ctl); }
__device__ __forceinline__ void rq_publish(int* en, unsigned ticket, int task, int stage,
                                           int kind, int domain) {
  proto::rq_publish<DevPlat>(en, ticket, task, stage, kind, domain);
}
__device__ __forceinline__ int rq_wait_ready(const int* en, unsigned h) {
  return proto::rq_wait_ready<DevPlat>(en, h);
}
__device__ __forceinline__ void rq_release(unsigned* ctl, int* en, unsigned h, unsigned cap) {
  proto::rq_release<DevPlat>(ctl, en, h, cap);
}

// ---------------------------------------------------------------------------
// The ring protocol of every stage loop here. GROUP = 1 (NS = 3 slots, one
// barrier per k-stage):
//   prologue  issue(0), issue(1)
//   stage s   wait until stage s has landed (stage s+1 may stay in flight);
//             lds_sync: stage s is visible to every wave, and every wave has
//             finished computing stage s-1, so its slot, (s+2) % 3, is free;
//             compute(s), with issue(s+2) folded in after its first reads.
// GROUP = 2 (NS = 4 slots in two halves, one barrier per pair of stages):
//   prologue  issue(0), issue(1)
//   pair s    (s even) wait until stages s and s+1 have landed (nothing else
//             is in flight); lds_sync: both visible, and every wave has
//             finished the previous pair, so the other half is free;
//             compute(s, s+1) as one group, with issue(s+2) and issue(s+3)
//             folded in. A tile of odd length S ends with the pair (S-1, S),
//             stage S all zeros.
//   end       wait for every load, lds_sync before the ring is used for
//             anything else.
// Every stage issues its LOADS loads, also past the tile's end: issue(t) for
// t >= S fills a free slot that nothing reads (a refetch of stage S-1), or,
// for GROUP = 2, with zeros that the second half of a tile's last pair may
// be computed on. So the loops carry no branch per load, and the wait at the top is always
// the same: vmcnt <= LOADS for GROUP = 1 (exactly the loads of stage s+1,
// and nothing a wave must read, were issued after stage s's; vmcnt retires
// in issue order), vmcnt = 0 for GROUP = 2.
template <class E>
__device__ __forceinline__ int next_slot(int slot) { return slot + 1 == E::NS ? 0 : slot + 1; }
__device__ __forceinline__ int slot_after_next(int slot) { return slot == 0 ? 2 : slot - 1; }
// This wave's 1 KiB piece of ring slot 0 (the LDS base of its stage loads),
// formed once per kernel.
__device__ __forceinline__ uint32_t wave_lds(const char* ring) {
  return pinned_sgpr((uint32_t)__builtin_amdgcn_readfirstlane(
      (int)(lds_addr_of(ring) + (uint32_t)(wave_id() * 1024))));
}
template <class E>
__device__ __forceinline__ void issue_loads(const typename E::Ctx& c, const typename E::Lane& ln,
                                            const typename E::Dst& d) {
#pragma unroll
  for (int i = 0; i < E::LOADS; ++i) E::issue_one(c, ln, d, i);
}
template <class E>
__device__ __forceinline__ void wait_landed() {
  static_assert((E::GROUP == 1 && E::NS == 3) || (E::GROUP == 2 && E::NS == 4), "ring shape");
  if constexpr (E::GROUP == 1) wait_vmcnt<E::LOADS>();
  else wait_vmcnt<0>();
}
// Load i (< GROUP * LOADS) of the next group's stages: d0 for the first
// stage, d1 for the second.
// The multiple of K (and of an urgent GEMM's K) an engine's tiles need:
// E::K_ALIGN where the engine states one (a load region spanning two
// stages), else one stage.
template <class E, class = void>
struct KAlign {
  static constexpr int value = E::KS;
};
template <class E>
struct KAlign<E, std::void_t<decltype(E::K_ALIGN)>> {
  static constexpr int value = E::K_ALIGN;
};

// An engine whose loads do not map one to one onto stages (a load region
// spanning both stages of a group) supplies its own E::issue_group.
template <class E, class = void>
struct HasIssueGroup {
  static constexpr bool value = false;
};
template <class E>
struct HasIssueGroup<E, std::void_t<decltype(&E::issue_group)>> {
  static constexpr bool value = true;
};
// An engine whose pairs are software-pipelined across the barrier
// (E::compute_pl, E::finish_tail): the stage loops carry its deferred k-step
// operands (TailFrag) from one pair to the next.
template <class E, class = void>
struct HasTailPipe {
  static constexpr bool value = false;
};
template <class E>
struct HasTailPipe<E, std::void_t<decltype(&E::finish_tail)>> {
  static constexpr bool value = true;
};
template <class E, bool = HasTailPipe<E>::value>
struct TailFrag {
  struct type {};
};
template <class E>
struct TailFrag<E, true> {
  using type = typename E::Tail;
};
// Whether the stage loops use it: for a tile whose block holds every wave of
// its SIMDs (one block per CU). With two blocks per CU the other block's
// wave already fills the idle stretch after a barrier (measured: no change
// at 2 and 4 blocks per CU).
template <class E, bool = HasTailPipe<E>::value>
struct PipelinedPairs {
  static constexpr bool value = false;
};
template <class E>
struct PipelinedPairs<E, true> {
  static constexpr bool value = E::BLOCKS_PER_CU == 1;
};
template <class E>
__device__ __forceinline__ void issue_group_one(const typename E::Ctx& c,
                                                const typename E::Lane& ln,
                                                const typename E::Dst& d0,
                                                const typename E::Dst& d1, int i) {
  if constexpr (HasIssueGroup<E>::value) {
    E::issue_group(c, ln, d0, d1, i);
  } else {
    if (i < E::LOADS) E::issue_one(c, ln, d0, i);
    else E::issue_one(c, ln, d1, i - E::LOADS);
  }
}

// Non-preemptible K loop over stages [0, S) of one tile. hook(s) runs
// uniformly before stage s is computed.
template <class E, class Hook>
__device__ __forceinline__ void run_stages(char* ring, uint32_t wl, const typename E::Ctx& c,
                                           typename E::Acc& acc, int row0, int col0, int S,
                                           Hook&& hook) {
  const typename E::Lane ln = E::lane_offsets(c, row0, col0);
  issue_loads<E>(c, ln, E::stage_dst(wl, c, 0, 0, S));
  issue_loads<E>(c, ln, E::stage_dst(wl, c, 1, 1, S));
  int slot = 0;
  // Pairs pipelined across the barrier (E::compute_pl), as in the
  // preemptible kernel with polls off.
  constexpr bool kPipe = PipelinedPairs<E>::value;
  typename TailFrag<E>::type tail;
  bool hasTail = false;
  for (int s = 0; s < S; s += E::GROUP) {
    hook(s);
    if constexpr (E::GROUP == 1) {
      wait_landed<E>();
      lds_sync();
      const typename E::Dst d = E::stage_dst(wl, c, slot_after_next(slot), s + 2, S);
      E::compute(ring, slot, acc, [] { return true; },
                 [&](int i) { E::issue_one(c, ln, d, i); });
      slot = next_slot<E>(slot);
    } else {
      // The next pair's load descriptors are formed and pinned before the
      // wait, so that nothing scalar stands between the barrier and the
      // next pair's loads (as in the preemptible kernel's pair loop).
      const int other = slot ^ 2;
      typename E::Dst d0 = E::stage_dst(wl, c, other, s + 2, S);
      typename E::Dst d1 = E::stage_dst(wl, c, other + 1, s + 3, S);
      E::pin(d0);
      if constexpr (!HasIssueGroup<E>::value) E::pin(d1);  // unused by region loads
      wait_landed<E>();
      lds_sync();
      if (s + 1 < S) hook(s + 1);
      auto mid = [&](int i) { issue_group_one<E>(c, ln, d0, d1, i); };
      if constexpr (kPipe) {
        E::compute_pl(ring, slot, acc, tail, hasTail, true, [] { return true; }, mid);
        hasTail = true;
      } else {
        E::compute(ring, slot, acc, [] { return true; }, mid);
      }
      slot = other;
    }
  }
  if constexpr (kPipe) {
    if (hasTail) E::finish_tail(acc, tail);
  }
  wait_vmcnt<0>();
  lds_sync();
}

// ---------------------------------------------------------------------------
// Flag sampling. Lane 0 of wave 0 loads the flag dword straight into LDS
// with a buffer load, so the sample rides the same in-order vmcnt stream as
// the stage data and lands no later than the stage wait that follows it: no
// wave ever stalls on the flag's cross-XCD round trip. Agent scope is sc1;
// a host-mapped flag is read at system scope (sc0 sc1). The other waves read
// the sample from LDS after the next barrier.
template <bool SYSTEM>
__device__ __forceinline__ void sample_flag(i32x4 flag_rsrc, uint32_t lds_addr) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_addr);
  const uint32_t zero = 0;
  if (threadIdx.x == 0) {
    if (SYSTEM)
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen sc0 sc1 lds"
                   : : "s"(m0), "v"(zero), "s"(flag_rsrc) : "memory");
    else
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen sc1 lds"
                   : : "s"(m0), "v"(zero), "s"(flag_rsrc) : "memory");
  }
}

// ---------------------------------------------------------------------------
// Bit-exact tile fingerprint: wrapping sum over the tile's elements of
// mix64(bits + (e << 32)), e = row*TN + col inside the tile. Sum order does
// not matter, so each thread hashes its own accumulators and the block
// reduces. The CPU oracle computes the same definition.

// Epilogue through LDS, in E::STORE_PASSES passes: each pass stages
// E::PASS_ROWS rows of the tile row-major in LDS (row stride E::STAGE_LD
// floats; LDS row rr is tile row E::pass_row(p, rr)), then every thread moves
// 16-byte pieces to C (coalesced rows) and, when asked, folds them into the
// fingerprint. Returns the per-thread partial hash. The caller must have
// finished every read of the ring (lds_sync) before calling.
template <class E, class = void>
struct HasDirectStore {
  static constexpr bool value = false;
};
template <class E>
struct HasDirectStore<E, std::void_t<decltype(&E::store_direct)>> {
  static constexpr bool value = true;
};
template <class E>
__device__ __forceinline__ uint64_t store_tile(const typename E::Acc& acc, char* lds,
                                               float* C, int ldc, int row0, int col0,
                                               bool want_hash) {
  // An engine whose accumulator layout holds whole row segments per register
  // stores an unfingerprinted tile directly (no LDS, no barrier).
  if constexpr (HasDirectStore<E>::value) {
    if (!want_hash) {
      E::store_direct(acc, C, ldc, row0, col0);
      return 0;
    }
  }
  uint64_t h = 0;
  constexpr int Q = E::TN / 4;  // float4 per row
  // Every thread moves the same number of float4 per pass, in batches of up
  // to 4 whose LDS reads are all issued before the batch's first store (one
  // read per store, each waited for in turn, serialised an LDS round trip
  // per float4: 16 of them per pass for a one-wave block, ~5 us per tile).
  // The batch loop stays rolled: unrolled, the 2-wave-per-SIMD polled
  // kernels took all 256 registers of their half of a SIMD, and a small
  // kernel on another stream (the retreat arm's flag raise) could no longer
  // be dispatched beside the grid.
  constexpr int ITERS = E::PASS_ROWS * Q / E::THREADS;
  constexpr int BATCH = ITERS < 4 ? ITERS : 4;
  static_assert(ITERS * E::THREADS == E::PASS_ROWS * Q && ITERS % BATCH == 0,
                "whole float4 per thread per pass");
#pragma unroll
  for (int p = 0; p < E::STORE_PASSES; ++p) {
    E::stage_pass(acc, lds, p);
    lds_sync();
#pragma unroll 1
    for (int b0 = 0; b0 < ITERS; b0 += BATCH) {
      float4 vs[BATCH];
#pragma unroll
      for (int it = 0; it < BATCH; ++it) {
        const int i = (int)threadIdx.x + (b0 + it) * E::THREADS;
        vs[it] = *(const float4*)((const float*)lds + (i / Q) * E::STAGE_LD + (i % Q) * 4);
      }
#pragma unroll
      for (int it = 0; it < BATCH; ++it) {
        const int i = (int)threadIdx.x + (b0 + it) * E::THREADS;
        const int r = E::pass_row(p, i / Q);
        *(float4*)(C + (size_t)(row0 + r) * ldc + col0 + (i % Q) * 4) = vs[it];
      }
    }
    // The fingerprint reads the pass again, one float4 at a time: hashed
    // under the unrolled stores, the 64-bit mixing of every value of the
    // pass at once spilled the polled kernels' registers.
    if (want_hash) {
#pragma unroll 1
      for (int it = 0; it < ITERS; ++it) {
        const int i = (int)threadIdx.x + it * E::THREADS;
        const int rr = i / Q, c4 = (i % Q) * 4;
        const int r = E::pass_row(p, rr);
        const float4 v = *(const float4*)((const float*)lds + rr * E::STAGE_LD + c4);
        const uint64_t e = (uint64_t)(r * E::TN + c4);
        h += mix64((uint64_t)__float_as_uint(v.x) + (e << 32));
        h += mix64((uint64_t)__float_as_uint(v.y) + ((e + 1) << 32));
        h += mix64((uint64_t)__float_as_uint(v.z) + ((e + 2) << 32));
        h += mix64((uint64_t)__float_as_uint(v.w) + ((e + 3) << 32));
      }
    }
    lds_sync();  // LDS reads done before the next pass or the ring refill
  }
  return h;
}

// Sum a per-thread uint64 over the block; valid in thread 0. `red` holds
// one slot per wave. Must be called by every thread.
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), off, 64);
    v += ((uint64_t)hi << 32) | lo;
  }
  if (lane_id() == 0) red[threadIdx.x >> 6] = v;
  lds_sync();
  uint64_t t = 0;
  if (threadIdx.x == 0)
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += red[w];
  lds_sync();
  return t;
}

// ---------------------------------------------------------------------------
// Checkpoint slot layout (per slot, floats):
//   [0, ACC_PER_THREAD*THREADS)        accumulators: float4 j of thread t at
//                                      (j*THREADS + t)*4 -> coalesced 16 B/lane
//   [ACC.., ACC.. + NS*STAGE/4)        the live stages s, s+1, ... of the ring
//                                      (positions 0, 1, ...), byte for byte: two
//                                      at a stage site, up to NS at an issue
//                                      site
template <class E>
struct Ckpt {
  static constexpr int ACC_FLOATS = E::ACC_PER_THREAD * E::THREADS;
  static constexpr int RING_FLOATS = E::NS * E::STAGE / 4;
  static constexpr int SLOT_FLOATS = ACC_FLOATS + RING_FLOATS;

  // Buffer stores/loads: one lane offset register, the float4 index in the
  // scalar offset, so the checkpoint adds no live address registers.
  // Both move the accumulators in groups of GROUP float4 per lane with a
  // scheduling barrier between groups: left free, the scheduler hoists every
  // accumulator read (or every load) to the top, which needs 4 VGPRs per
  // float4 at once -- all 256 VGPRs for the bf16 tile -- and spills.
  static constexpr int NJ = E::ACC_PER_THREAD / 4, GROUP = NJ < 8 ? NJ : 8;
  // CPOL_SC1 for a checkpoint another XCD reads back (the retreat arm's
  // resume slots): written through, published without an L2 write-back.
  template <int CPOL = 0>
  static __device__ __forceinline__ void save_acc(const typename E::Acc& a, float* slot) {
    const buf_rsrc r = make_buf_rsrc(slot, ACC_FLOATS * 4);
    const int vo = (int)threadIdx.x * 16;
#pragma unroll
    for (int j0 = 0; j0 < NJ; j0 += GROUP) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = j0; j < j0 + GROUP; ++j) {
        const float4 v = {E::get(a, 4 * j), E::get(a, 4 * j + 1), E::get(a, 4 * j + 2),
                          E::get(a, 4 * j + 3)};
        buf_store_f4<CPOL>(v, r, vo, j * E::THREADS * 16);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  static __device__ __forceinline__ void load_acc(typename E::Acc& a, const float* slot) {
    const buf_rsrc r = make_buf_rsrc(slot, ACC_FLOATS * 4);
    const int vo = (int)threadIdx.x * 16;
#pragma unroll
    for (int j0 = 0; j0 < NJ; j0 += GROUP) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = j0; j < j0 + GROUP; ++j) {
        const float4 v = buf_load_f4(r, vo, j * E::THREADS * 16);
        E::set(a, 4 * j, v.x);
        E::set(a, 4 * j + 1, v.y);
        E::set(a, 4 * j + 2, v.z);
        E::set(a, 4 * j + 3, v.w);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // Retire the loads here, on the rare restore path. Otherwise the
    // compiler's wait insertion sees loads still pending into the
    // accumulator registers where the restore path rejoins the stage loop and
    // puts vmcnt waits at the head of the shared compute block -- which then
    // drain the prefetched stages on every k-stage of every tile.
    wait_vmcnt<0>();
  }
  // Copy n (<= NS) ring slots first, first+1, ... (mod NS) to / from
  // checkpoint positions 0, 1, ...
  // save_ring copies the newest stage (position n-1) first: without a drain
  // it is the one whose loads may still be landing.
  template <int CPOL = 0>
  static __device__ __forceinline__ void save_ring(const char* ring, float* slot,
                                                   int first, int n) {
    const buf_rsrc r = make_buf_rsrc(slot + ACC_FLOATS, RING_FLOATS * 4);
    for (int k = n - 1; k >= 0; --k) {
      const int b = (first + k) % E::NS;
      for (int i = threadIdx.x * 16; i < E::STAGE; i += E::THREADS * 16)
        buf_store_f4<CPOL>(*(const float4*)(ring + b * E::STAGE + i), r, i, k * E::STAGE);
    }
  }
  static __device__ __forceinline__ void load_ring(char* ring, const float* slot,
                                                   int first, int n) {
    const char* src = (const char*)(slot + ACC_FLOATS);
    for (int k = 0; k < n; ++k) {
      const int b = (first + k) % E::NS;
      for (int i = threadIdx.x * 16; i < E::STAGE; i += E::THREADS * 16)
        *(float4*)(ring + b * E::STAGE + i) = *(const float4*)(src + k * E::STAGE + i);
    }
  }
  // Whether any of the 16-byte pieces this thread saved with save_ring
  // (same first, n) differs from the ring as it stands now. Call after every
  // load into the ring has landed and the thread's own checkpoint stores
  // have completed.
  static __device__ __forceinline__ bool ring_differs(const char* ring, const float* slot,
                                                      int first, int n) {
    const char* src = (const char*)(slot + ACC_FLOATS);
    bool d = false;
    for (int k = 0; k < n; ++k) {
      const int b = (first + k) % E::NS;
      for (int i = threadIdx.x * 16; i < E::STAGE; i += E::THREADS * 16) {
        const uint4 x = *(const uint4*)(ring + b * E::STAGE + i);
        const uint4 y = *(const uint4*)(src + k * E::STAGE + i);
        d |= (x.x != y.x) | (x.y != y.y) | (x.z != y.z) | (x.w != y.w);
      }
    }
    return d;
  }
};

// This thread's 16 bytes of the last direct-to-LDS load of the stage in ring
// slot `sl`, read as they stand (a load still in flight has not yet written
// them). The read completes before the function returns.
template <class E>
__device__ __forceinline__ uint4 probe_last_load(const char* ring, int sl) {
  const volatile uint4* p = (const volatile uint4*)(ring + sl * E::STAGE +
                                                    E::dma_lds_off(E::LOADS - 1) +
                                                    16 * threadIdx.x);
  const uint4 v = {p->x, p->y, p->z, p->w};
  wait_lgkmcnt0();
  asm volatile("" ::: "memory");
  return v;
}

}  // namespace apk
