// engine_valu64.hpp -- the reference's 64x64 fp32 SGEMM tile semantics on
// gfx950 vector ALUs: every output is one fmaf chain over k in ascending order
// (reference src/tile.cuh:62-107), so the result is bit-identical to a
// correctly rounded sequential fmaf on the host.
//
// Block: 256 threads = 4 wave64s; thread (tx = t%16, ty = t/16) owns the 4x4
// outputs rows ty*4..+3, cols tx*4..+3 (the reference's mapping).
// Stage: k depth KS=32, A stage 64x32 fp32 (8 KiB) + B stage 32x64 fp32
// (8 KiB), filled by buffer_load_dwordx4 ... lds into a 3-slot ring (48 KiB).
//
// LDS layouts:
//  A stage: 64 rows x 128 B. 16-byte quad q of row r sits at slot
//           q ^ ((r >> 2) & 7). One read instruction of a wave touches the
//           four rows r, r+4, r+8, r+12 (one per ty of the wave); the swizzle
//           gives them four different slots, hence different banks.
//  B stage: 32 rows x 256 B, natural; B[kk][tx*4..+3] is one 16-byte read
//           per lane, 16 lanes covering 256 contiguous bytes.
#pragma once
#include "device.hpp"

namespace apk {

struct EngValu64 {
  static constexpr int TM = 64, TN = 64, KS = 32, NS = 3, GROUP = 1, THREADS = 256;
  // Waves per SIMD at most (3 blocks per CU (LDS-bound)): the register budget the
  // compiler may schedule for.
  static constexpr int WAVES_PER_SIMD = 3;
  static constexpr int MIN_WAVES_PER_SIMD = 1;  // occupancy the registers must allow
  static constexpr int A_STAGE = TM * KS * 4;               // 8 KiB
  static constexpr int B_STAGE = KS * TN * 4;               // 8 KiB
  static constexpr int STAGE = A_STAGE + B_STAGE;           // 16 KiB
  static constexpr int LDS_BYTES = NS * STAGE;              // 48 KiB
  static constexpr int LOADS_A = A_STAGE / (THREADS * 16);  // 2
  static constexpr int LOADS_B = B_STAGE / (THREADS * 16);  // 2
  static constexpr int LOADS = LOADS_A + LOADS_B;
  static constexpr int ACC_PER_THREAD = 16;                 // floats
  static constexpr int ELEM_BYTES = 4;                      // fp32 operands
  // Epilogue: the whole tile is staged in LDS in one pass (row stride TN).
  static constexpr int STORE_PASSES = 1, PASS_ROWS = TM, STAGE_LD = TN;

  struct Acc {
    float v[4][4];
  };

  struct Ctx {
    i32x4 ra, rb;
    int K, N;
  };

  static __device__ __forceinline__ Ctx make_ctx(const void* A, const void* B,
                                                 int M, int N, int K) {
    Ctx c;
    c.ra = make_rsrc(A, (uint32_t)((size_t)M * K * 4));
    c.rb = make_rsrc(B, (uint32_t)((size_t)K * N * 4));
    c.K = K;
    c.N = N;
    return c;
  }

  static __device__ __forceinline__ void zero(Acc& a) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) a.v[i][j] = 0.0f;
  }

  static __device__ __forceinline__ int aswz(int r) { return (r >> 2) & 7; }

  // Direct-to-LDS loads of one k-stage. A load i (< 2) fills the 1 KiB
  // piece i*4 + wave of the A stage: rows 32*i + 8*wave + lane/8, quad slot
  // lane%8; B load i fills rows 16*i + 4*wave + lane/16. The A swizzle uses
  // row bits 2-4 only, so each lane's offset of load i is fixed per tile
  // (Lane, one register per load) and stage s only adds scalar offsets.
  struct Lane {
    uint32_t a[LOADS_A], b[LOADS_B];
  };
  static __device__ __forceinline__ Lane lane_offsets(const Ctx& c, int row0, int col0) {
    const int w = wave_id(), l = lane_id();
    const int ra = w * 8 + (l >> 3);
    const int qa = (l & 7) ^ aswz(ra);
    const int rb = w * 4 + (l >> 4);
    const uint32_t a0 = (uint32_t)(((row0 + ra) * c.K + 4 * qa) * 4);
    const uint32_t b0 = (uint32_t)((rb * c.N + col0 + 4 * (l & 15)) * 4);
    Lane ln;
#pragma unroll
    for (int i = 0; i < LOADS_A; ++i) ln.a[i] = a0 + (uint32_t)(i * 32) * (uint32_t)c.K * 4u;
#pragma unroll
    for (int i = 0; i < LOADS_B; ++i) ln.b[i] = b0 + (uint32_t)(i * 16) * (uint32_t)c.N * 4u;
    return ln;
  }
  // The scalar parts of the loads of stage t into ring slot `slot`, formed
  // once per stage: this wave's 1 KiB piece of the slot (LDS; wave_lds is
  // the piece in slot 0) and the byte offsets of k-stage t in A (along a
  // row) and B (down the rows).
  struct Dst {
    uint32_t lds, ka, kb;
  };
  // A stage past the tile's end (t >= S) fetches stage S-1 again: nothing
  // reads that slot before it is refilled.
  static __device__ __forceinline__ Dst stage_dst(uint32_t wave_lds, const Ctx& c, int slot,
                                                  int t, int S) {
    const uint32_t k0 = (uint32_t)((t < S ? t : S - 1) * KS);
    return Dst{wave_lds + (uint32_t)(slot * STAGE), k0 * 4u, k0 * (uint32_t)c.N * 4u};
  }
  // Byte offset inside a ring slot of load i's piece: thread t's 16 bytes of
  // load i land at slot + dma_lds_off(i) + 16 t.
  static constexpr uint32_t dma_lds_off(int i) {
    return (uint32_t)(i < LOADS_A ? i * 4096 : A_STAGE + (i - LOADS_A) * 4096);
  }
  static __device__ __forceinline__ void issue_one(const Ctx& c, const Lane& ln, const Dst& d,
                                                   int i) {
    if (i < LOADS_A)
      dma_x4(c.ra, d.lds, dma_lds_off(i), ln.a[i], d.ka);
    else
      dma_x4(c.rb, d.lds, dma_lds_off(i), ln.b[i - LOADS_A], d.kb);
  }

  // One k-stage out of ring slot `slot`. `pre` runs first (flag check;
  // returning false abandons the stage before any accumulator changes),
  // `mid(i)` after k step i for i < LOADS (the next stage's direct-to-LDS
  // load i). The operands of k step kk+1 are read from LDS before the 16
  // FMAs of step kk are issued (a scheduling barrier keeps the compiler
  // from sinking each read next to its use, where one wave per SIMD would
  // wait out the LDS latency at every step); the FMA order is unchanged.
  struct Ops {
    float a[4];
    float4 b;
  };
  template <class Pre, class Mid>
  static __device__ __forceinline__ bool compute(const char* ring, int slot, Acc& acc,
                                                 Pre&& pre, Mid&& mid) {
    const char* abase = ring + slot * STAGE;
    const float* bs = (const float*)(abase + A_STAGE);
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    auto rd = [&](int kk, Ops& o) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = ty * 4 + i;
        const int slotq = (kk >> 2) ^ aswz(r);
        o.a[i] = *(const float*)(abase + r * 128 + slotq * 16 + (kk & 3) * 4);
      }
      o.b = *(const float4*)(bs + kk * TN + tx * 4);
    };
    if (!pre()) return false;
    Ops o[2];
    rd(0, o[0]);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      if (kk + 1 < KS) rd(kk + 1, o[(kk + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      const Ops& c = o[kk & 1];
      const float bb[4] = {c.b.x, c.b.y, c.b.z, c.b.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc.v[i][j] = fmaf(c.a[i], bb[j], acc.v[i][j]);
      if (kk < LOADS) {
        __builtin_amdgcn_sched_barrier(0);
        mid(kk);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    return true;
  }
  static __device__ __forceinline__ void compute(const char* ring, int slot, Acc& acc) {
    compute(ring, slot, acc, [] { return true; }, [](int) {});
  }

  // Output element (tile-relative row, col) of accumulator register e.
  static __device__ __forceinline__ void coord(int e, int& r, int& c) {
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    r = ty * 4 + (e >> 2);
    c = tx * 4 + (e & 3);
  }
  static __device__ __forceinline__ float get(const Acc& a, int e) {
    return a.v[e >> 2][e & 3];
  }
  static __device__ __forceinline__ void set(Acc& a, int e, float v) {
    a.v[e >> 2][e & 3] = v;
  }

  // Write the accumulators into LDS as the row-major TM x TN tile.
  static __device__ __forceinline__ int pass_row(int, int rr) { return rr; }
  static __device__ __forceinline__ void stage_pass(const Acc& acc, char* lds, int) {
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    float* t = (float*)lds;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 v = {acc.v[i][0], acc.v[i][1], acc.v[i][2], acc.v[i][3]};
      *(float4*)(t + (ty * 4 + i) * TN + tx * 4) = v;
    }
  }
};

}  // namespace apk
