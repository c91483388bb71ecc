// device.hpp -- gfx950 device primitives shared by every persistent kernel:
// the flag contract, the work-queue atomic, timers, LDS-only barriers,
// explicit vmcnt waits and buffer-resource direct-to-LDS loads.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "apk.h"

namespace apk {

// ---------------------------------------------------------------------------
// Flag contract (reference src/tile.cuh:15-30): the generation flag carries
// only its value; nothing is published through it. Loads and stores are
// relaxed and agent-scope, so the value is coherent across the 8 XCD L2s
// (the load compiles to `global_load_dword ... sc1`).
__device__ __forceinline__ int flag_load(const int* f) {
  return __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void flag_store(int* f, int v) {
  __hip_atomic_store(f, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned fetch_add_u32(unsigned* p, unsigned v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int fetch_add_i32(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void atomic_max_u64(unsigned long long* p,
                                               unsigned long long v) {
  __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void atomic_min_i64(long long* p, long long v) {
  __hip_atomic_fetch_min(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void atomic_max_i64(long long* p, long long v) {
  __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Timers. wall_ticks() is s_memrealtime: a constant-rate counter shared by
// all CUs and XCDs (rate from hipDeviceAttributeWallClockRate, 100 MHz on
// MI355X), the analog of %globaltimer (reference src/tile.cuh:50-57).
// hw_slot() encodes XCC, SE and CU of the executing wave (the %smid analog,
// src/tile.cuh:44-48).
__device__ __forceinline__ int64_t wall_ticks() { return (int64_t)wall_clock64(); }
__device__ __forceinline__ unsigned hw_slot() { return __smid(); }
// The XCD (XCC) the executing wave runs on, 0..7 on MI355X: hardware
// register XCC_ID (20), bits [3:0] -> s_getreg_b32 immediate
// size-1 = 3 << 11 | offset 0 << 6 | 20.
__device__ __forceinline__ unsigned xcc_id() {
  return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & (APK_QUEUE_XCDS - 1);
}
// The shader engine (0..3) of the executing wave inside its XCD: hardware
// register HW_ID (4), SE_ID bits [14:13] -> size-1 = 1, offset 13.
__device__ __forceinline__ unsigned se_id() {
  return __builtin_amdgcn_s_getreg((1 << 11) | (13 << 6) | 4) & (APK_SES_PER_XCD - 1);
}

// ---------------------------------------------------------------------------
// Barriers. __syncthreads() carries a workgroup release/acquire fence, which
// on gfx950 waits vmcnt(0) and would drain every in-flight direct-to-LDS
// load. lds_sync() fences only LDS (lgkmcnt) and then barriers, so a
// software pipeline keeps its prefetches in flight across it. Waits for the
// prefetched data itself are explicit (wait_vmcnt).
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] in bits 3:0 and vmcnt[5:4] in bits 15:14; expcnt=7 and
// lgkmcnt=15 mean "no wait" for those counters).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(0) alone (vmcnt 63 and expcnt 7 mean "no wait").
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
}

// ---------------------------------------------------------------------------
// Buffer resources and direct-to-LDS loads. A raw buffer with stride 0
// returns zero for loads beyond num_records bytes instead of touching
// memory, so a direct-to-LDS load can never fault even if a tile coordinate
// were wrong. dword3 = 0x00020000 is the gfx9 raw 32-bit data format.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  i32x4 r;
  r.x = (int)(uint32_t)(a & 0xffffffffu);
  r.y = (int)(uint32_t)(a >> 32);  // stride 0
  r.z = (int)bytes;
  r.w = 0x00020000;
  return r;
}

// Compiler-visible buffer loads/stores (tracked by the wait-insertion pass,
// unlike the direct-to-LDS asm below): wave-uniform base in the resource,
// per-lane byte offset in a VGPR, a uniform byte offset in an SGPR.
typedef __amdgpu_buffer_rsrc_t buf_rsrc;
__device__ __forceinline__ buf_rsrc make_buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
// CPOL: the store's cache policy; CPOL_SC1 (agent coherence) writes the line
// through this XCD's L2, so the data is visible device-wide once the store
// has completed (vmcnt), with no write-back of the whole L2 (a release fence
// at agent scope is one: buffer_wbl2 sc1).
constexpr int CPOL_SC1 = 16;
template <int CPOL = 0>
__device__ __forceinline__ void buf_store_f4(float4 v, buf_rsrc r, int voff, int soff) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 u = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                   __float_as_uint(v.w)};
  __builtin_amdgcn_raw_buffer_store_b128(u, r, voff, soff, CPOL);
}
__device__ __forceinline__ float4 buf_load_f4(buf_rsrc r, int voff, int soff) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                     __uint_as_float(u.w));
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// splitmix64 finaliser: the mixing step of the tile fingerprints.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// 32-bit LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr_of(const void* p) {
  return (uint32_t)(uintptr_t)((__attribute__((address_space(3))) const void*)p);
}
// Index of the executing wave in its block, as a scalar.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}
// Direct-to-LDS 16-byte-per-lane buffer load with every address part but
// the lane offset kept scalar: lane l's bytes land at LDS address
// lds + off + 16*l, read from base + soff + voff. `off` must fold to a
// compile-time constant (the load's place in a stage): M0 is then formed by
// one scalar add, the only scalar instruction a load costs in the stage loops.
__device__ __forceinline__ void dma_x4(i32x4 rsrc, uint32_t lds, uint32_t off, uint32_t voff,
                                       uint32_t soff) {
  asm volatile("s_add_u32 m0, %0, %1\n\tbuffer_load_dwordx4 %2, %3, %4 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "i"(off), "v"(voff), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane(soff))
               : "memory", "scc");
}
// A scalar the optimiser must keep as computed: it can neither recompute it
// at every use (as it would a readfirstlane of a thread-id expression inside
// a loop) nor fold it into its uses.
__device__ __forceinline__ uint32_t pinned_sgpr(uint32_t v) {
  asm volatile("" : "+s"(v));
  return v;
}

// One 16-byte-per-lane buffer load written straight into LDS: lane l's 16
// bytes land at lds_base + 16*l (lds_base is wave-uniform, passed in M0).
//
// Issued as inline asm on purpose: the compiler's waitcnt pass cannot tell
// which LDS bytes a DMA load writes when the ring slot is chosen at run
// time, so with the builtin it puts vmcnt(0) before every LDS read and the
// prefetch pipeline collapses. Kernels here wait for their DMA data
// explicitly (wait_vmcnt + lds_sync), and the pass only ever over-waits for
// its own loads because these DMA loads are invisible to its count. M0 holds
// no long-lived value on gfx9+ (LDS instructions do not read it), so setting
// it here is local to the asm.
__device__ __forceinline__ void load_lds_x4(i32x4 rsrc, const void* lds_base,
                                            uint32_t voffset_bytes) {
  const uint32_t lds_addr = (uint32_t)(uintptr_t)(
      (__attribute__((address_space(3))) const void*)lds_base);
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voffset_bytes),
        "s"(rsrc)
      : "memory");
}

// The kernel's explicit arguments, read in place in the kernel-argument
// segment (they start at its offset 0) through a pointer the optimiser cannot
// see through: loads through it are neither hoisted above the point of use
// nor merged with earlier ones. Kernels with many parameters read them this
// way where they are used, so the compiler does not load every parameter at
// entry and keep them all live in scalar registers (where they spill into
// vector registers). Taking the address of a by-value kernel parameter
// instead would copy the whole struct to scratch memory.
template <class T>
using KArg = __attribute__((address_space(4))) const T;
template <class T>
__device__ __forceinline__ KArg<T>* kernel_args() {
  KArg<T>* p = (KArg<T>*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return p;
}

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

// A value every lane of the block holds identically (read from LDS after a
// barrier), made scalar for the compiler. Loop exits and branches that
// enclose barriers must be taken on such values: if the compiler sees a
// per-lane (VGPR) condition it may structurize the loop as a divergent one,
// park some lanes of a wave outside an inner loop and let the others run
// through barriers on their own -- a block that deadlocks or livelocks even
// though the value was uniform at run time.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ unsigned uniform(unsigned v) {
  return (unsigned)__builtin_amdgcn_readfirstlane((int)v);
}

}  // namespace apk
