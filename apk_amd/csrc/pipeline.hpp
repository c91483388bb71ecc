// pipeline.hpp -- engine-independent pieces of the persistent kernels:
// the 3-slot direct-to-LDS software pipeline, flag sampling through LDS, the
// bit-exact tile fingerprint, and checkpoint save/restore of accumulators and
// LDS stages.
#pragma once
#include "device.hpp"

namespace apk {

// Prefetch depth of every ring here: NS = 3 slots, P = 2 stages in flight.
constexpr int kPrefetch = 2;

// Wait until k-stage s has landed when `ahead` (0..2) later stages were
// issued behind it, each stage being E::LOADS + EXTRA vector-memory
// operations per wave (EXTRA = 1 when a flag sample rides with the stage).
// vmcnt retires in issue order, so <= ahead*(LOADS+EXTRA) outstanding
// operations means stage s is in LDS. More operations issued later (stores,
// atomics) only make the wait stricter, never wrong.
template <class E, int EXTRA>
__device__ __forceinline__ void wait_stage(int ahead) {
  static_assert(E::NS == kPrefetch + 1, "ring of 3");
  if (ahead >= 2) wait_vmcnt<2 * (E::LOADS + EXTRA)>();
  else if (ahead == 1) wait_vmcnt<E::LOADS + EXTRA>();
  else wait_vmcnt<0>();
}

// Wait until at most n vector-memory operations of this wave are
// outstanding, for the n a ring can produce: 0, L, L+1, 2L, 2L+1, 2L+2 (L =
// E::LOADS per stage, +1 per stage that carries a flag sample). Any other n
// waits for everything, which is always safe.
template <class E>
__device__ __forceinline__ void wait_ops(int n) {
  constexpr int L = E::LOADS;
  if (n == 2 * L + 2) wait_vmcnt<2 * L + 2>();
  else if (n == 2 * L + 1) wait_vmcnt<2 * L + 1>();
  else if (n == 2 * L) wait_vmcnt<2 * L>();
  else if (n == L + 1) wait_vmcnt<L + 1>();
  else if (n == L) wait_vmcnt<L>();
  else wait_vmcnt<0>();
}

// Non-preemptible K loop over stages [0, S) of one tile: prologue of two
// stages, then issue s+2 / wait s / compute s. hook(s) runs uniformly at the
// top of stage s.
template <class E, class Hook>
__device__ __forceinline__ void run_stages(char* ring, const typename E::Ctx& c,
                                           typename E::Acc& acc, int row0, int col0,
                                           int S, Hook&& hook) {
  if (S > 0) E::issue(ring, c, 0, row0, col0, 0);
  if (S > 1) E::issue(ring, c, 1, row0, col0, 1);
  for (int s = 0; s < S; ++s) {
    hook(s);
    if (s + kPrefetch < S) E::issue(ring, c, (s + kPrefetch) % E::NS, row0, col0, s + kPrefetch);
    wait_stage<E, 0>(S - 1 - s < kPrefetch ? S - 1 - s : kPrefetch);
    lds_sync();
    E::compute(ring, s % E::NS, acc);
    lds_sync();
  }
}

// ---------------------------------------------------------------------------
// Flag sampling. One dword is loaded from the flag straight into LDS by a
// buffer load, so the sample rides the same in-order vmcnt stream as the
// stage data and is read from LDS once a later stage wait has retired it: no
// wave ever stalls on the flag's cross-XCD round trip. Only wave 0's lane 0
// samples the real flag (agent scope: sc1, or system scope sc0 sc1 for a
// host-mapped flag); lanes 0 of waves 1..3 load a cached dword so that every
// wave has the same number of operations per stage.
template <bool SYSTEM>
__device__ __forceinline__ void sample_flag(i32x4 flag_rsrc, i32x4 dummy_rsrc,
                                            int* lds_dst_wave) {
  const uint32_t lds_addr = (uint32_t)(uintptr_t)(
      (__attribute__((address_space(3))) const void*)lds_dst_wave);
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_addr);
  const uint32_t zero = 0;
  if (lane_id() == 0) {
    if ((threadIdx.x >> 6) == 0) {
      if (SYSTEM)
        asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen sc0 sc1 lds"
                     : : "s"(m0), "v"(zero), "s"(flag_rsrc) : "memory");
      else
        asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen sc1 lds"
                     : : "s"(m0), "v"(zero), "s"(flag_rsrc) : "memory");
    } else {
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                   : : "s"(m0), "v"(zero), "s"(dummy_rsrc) : "memory");
    }
  }
}

// ---------------------------------------------------------------------------
// Bit-exact tile fingerprint: wrapping sum over the tile's elements of
// splitmix64(bits + (e << 32)), e = row*TN + col inside the tile. Sum order
// does not matter, so each thread hashes its own accumulators and the block
// reduces. The CPU oracle computes the same definition.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// Epilogue through LDS: the tile is staged row-major in LDS, then every
// thread moves 16-byte pieces to C (coalesced rows) and, when asked, folds
// them into the fingerprint. Returns the per-thread partial hash. The caller
// must have finished every read of the ring (lds_sync) before calling.
template <class E>
__device__ __forceinline__ uint64_t store_tile(const typename E::Acc& acc, char* lds,
                                               float* C, int ldc, int row0, int col0,
                                               bool want_hash) {
  E::stage_tile(acc, lds);
  lds_sync();
  uint64_t h = 0;
  const float4* t = (const float4*)lds;
  constexpr int Q = E::TN / 4;  // float4 per row
  for (int i = threadIdx.x; i < E::TM * Q; i += E::THREADS) {
    const int r = i / Q, c4 = (i % Q) * 4;
    const float4 v = t[i];
    *(float4*)(C + (size_t)(row0 + r) * ldc + col0 + c4) = v;
    if (want_hash) {
      const uint64_t e = (uint64_t)(r * E::TN + c4);
      h += mix64((uint64_t)__float_as_uint(v.x) + (e << 32));
      h += mix64((uint64_t)__float_as_uint(v.y) + ((e + 1) << 32));
      h += mix64((uint64_t)__float_as_uint(v.z) + ((e + 2) << 32));
      h += mix64((uint64_t)__float_as_uint(v.w) + ((e + 3) << 32));
    }
  }
  lds_sync();  // LDS reads done before the ring is refilled
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
//   [ACC.., ACC.. + NS*STAGE/4)        the LDS ring, byte for byte
template <class E>
struct Ckpt {
  static constexpr int ACC_FLOATS = E::ACC_PER_THREAD * E::THREADS;
  static constexpr int RING_FLOATS = E::LDS_BYTES / 4;
  static constexpr int SLOT_FLOATS = ACC_FLOATS + RING_FLOATS;

  static __device__ __forceinline__ void save_acc(const typename E::Acc& a, float* slot) {
#pragma unroll
    for (int j = 0; j < E::ACC_PER_THREAD / 4; ++j) {
      float4 v = {E::get(a, 4 * j), E::get(a, 4 * j + 1), E::get(a, 4 * j + 2),
                  E::get(a, 4 * j + 3)};
      *(float4*)(slot + ((size_t)j * E::THREADS + threadIdx.x) * 4) = v;
    }
  }
  static __device__ __forceinline__ void load_acc(typename E::Acc& a, const float* slot) {
#pragma unroll
    for (int j = 0; j < E::ACC_PER_THREAD / 4; ++j) {
      const float4 v = *(const float4*)(slot + ((size_t)j * E::THREADS + threadIdx.x) * 4);
      E::set(a, 4 * j, v.x);
      E::set(a, 4 * j + 1, v.y);
      E::set(a, 4 * j + 2, v.z);
      E::set(a, 4 * j + 3, v.w);
    }
  }
  // Copy ring slots [first, first+n) (mod NS) to / from the checkpoint.
  static __device__ __forceinline__ void save_ring(const char* ring, float* slot,
                                                   int first, int n) {
    char* dst = (char*)(slot + ACC_FLOATS);
    for (int k = 0; k < n; ++k) {
      const int b = (first + k) % E::NS;
      for (int i = threadIdx.x * 16; i < E::STAGE; i += E::THREADS * 16)
        *(float4*)(dst + b * E::STAGE + i) = *(const float4*)(ring + b * E::STAGE + i);
    }
  }
  static __device__ __forceinline__ void load_ring(char* ring, const float* slot,
                                                   int first, int n) {
    const char* src = (const char*)(slot + ACC_FLOATS);
    for (int k = 0; k < n; ++k) {
      const int b = (first + k) % E::NS;
      for (int i = threadIdx.x * 16; i < E::STAGE; i += E::THREADS * 16)
        *(float4*)(ring + b * E::STAGE + i) = *(const float4*)(src + b * E::STAGE + i);
    }
  }
};

}  // namespace apk
