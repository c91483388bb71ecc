// engine_mfma128.hpp -- 128x128 fp32 output tile on the gfx950 fp32 matrix
// cores (v_mfma_f32_32x32x2_f32), fed by a 3-stage LDS ring of
// buffer_load_dwordx4 ... lds (direct-to-LDS, no VGPR staging).
//
// Two ring shapes of the same tile (template parameter G):
//  G = 1 (EngMfma128): 3 slots, one barrier per k-stage -- the preemptible
//        kernels, which poll at every k-stage;
//  G = 2 (EngMfma128Pairs): 4 slots (128 KiB) taken in pairs of k-stages,
//        one barrier per pair -- the non-preemptible persistent GEMM and the
//        urgent-job kernel, for tiles of an even number of k-stages. With
//        one wave per SIMD nothing covers a barrier's wait and first operand
//        reads, so halving the barriers gains 1.5-2% (4096^3 and 8192^3,
//        ABAB).
// Both walk every output's k in the same order, so their C is bit-identical.
//
// Block: 256 threads = 4 wave64s in a 2x2 arrangement; each wave owns a
// 64x64 sub-tile held as 2x2 32x32 accumulators (64 VGPRs per lane).
// Stage: k depth KS=32 -> A stage 128x32 fp32 (16 KiB) + B stage 32x128 fp32
// (16 KiB); 3 stages = 96 KiB (pairs: 4 = 128 KiB) of the 160 KiB LDS (1 block
// per CU).
//
// LDS layouts (bank-conflict-free for the MFMA operand reads):
//  A stage: 128 rows x 128 B. 16-byte quad q of row r is stored at slot
//           q ^ aswz(r), aswz(r) = (r ^ ((r >> 3) & 1)) & 7: 8 (or 16)
//           consecutive rows reading the same quad hit 8 (16) different
//           16-byte bank groups, whether the LDS serves 128 B or 256 B per
//           cycle.
//  B stage: 32 rows x 512 B; 16-byte chunk c of row k is stored at slot
//           c ^ (((k >> 2) & 1) << 3). An operand read is 32 consecutive
//           dwords of row k for the lower half-wave and of row k+4 for the
//           upper one; the XOR moves the upper half by 128 B, so the two
//           halves never share a bank even when all 64 lanes are served in
//           one cycle.
//
// k order inside a stage: k-group g (8 values) is consumed in 4 MFMA steps;
// in step s the lower half-wave supplies k = 8g+s and the upper half-wave
// k = 8g+4+s. The order is fixed, so a tile's result is a deterministic
// function of its inputs whatever worker computes it and however often it
// is checkpointed and resumed.
#pragma once
#include "device.hpp"

namespace apk {

template <int G>
struct EngMfma128T {
  static_assert(G == 1 || G == 2, "stage groups of 1 or 2");
  static constexpr int TM = 128, TN = 128, KS = 32, NS = G == 2 ? 4 : 3, GROUP = G,
                       THREADS = 256;
  // Pairs take tiles of an even number of k-stages only (a stage past the
  // tile's end refetches the last one, which a pair would compute): the
  // launches pick the one-stage ring for the others.
  // Waves per SIMD at most (1 block per CU (LDS-bound)): the register budget the
  // compiler may schedule for.
  static constexpr int WAVES_PER_SIMD = 1;
  static constexpr int MIN_WAVES_PER_SIMD = 1;  // occupancy the registers must allow
  static constexpr int A_STAGE = TM * KS * 4;               // bytes
  static constexpr int B_STAGE = KS * TN * 4;               // bytes
  static constexpr int STAGE = A_STAGE + B_STAGE;           // 32 KiB
  static constexpr int LDS_BYTES = NS * STAGE;              // 96 / 128 KiB
  static constexpr int LOADS_A = A_STAGE / (THREADS * 16);  // 4 per thread
  static constexpr int LOADS_B = B_STAGE / (THREADS * 16);  // 4 per thread
  static constexpr int LOADS = LOADS_A + LOADS_B;           // per stage
  static constexpr int ACC_PER_THREAD = 64;                 // floats
  static constexpr int ELEM_BYTES = 4;                      // fp32 operands
  // Epilogue: the whole tile is staged in LDS in one pass (row stride TN).
  static constexpr int STORE_PASSES = 1, PASS_ROWS = TM, STAGE_LD = TN;

  struct Acc {
    f32x16 c[2][2];
  };

  static __device__ __forceinline__ int aswz(int r) { return (r ^ ((r >> 3) & 1)) & 7; }
  static __device__ __forceinline__ int bswz(int k) { return ((k >> 2) & 1) << 3; }

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
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) a.c[i][j][r] = 0.0f;
  }

  // Direct-to-LDS loads of one k-stage. A load i (< 4) fills the 1 KiB
  // piece i*4 + wave of the A stage: rows 32*i + 8*wave + lane/8, quad slot
  // lane%8. B load i fills rows 8*i + 2*wave + lane/32, chunk slot lane%32.
  // Neither swizzle depends on the row bits that i changes, so each lane's
  // offset of load i is fixed per tile (Lane, one register per load) and
  // stage s only adds scalar offsets.
  struct Lane {
    uint32_t a[LOADS_A], b[LOADS_B];
  };
  static __device__ __forceinline__ Lane lane_offsets(const Ctx& c, int row0, int col0) {
    const int w = wave_id(), l = lane_id();
    const int ra = w * 8 + (l >> 3);
    const int qa = (l & 7) ^ aswz(ra);
    const int rb = w * 2 + (l >> 5);
    const int cq = (l & 31) ^ bswz(rb);
    const uint32_t a0 = (uint32_t)(((row0 + ra) * c.K + 4 * qa) * 4);
    const uint32_t b0 = (uint32_t)((rb * c.N + col0 + 4 * cq) * 4);
    Lane ln;
#pragma unroll
    for (int i = 0; i < LOADS_A; ++i) ln.a[i] = a0 + (uint32_t)(i * 32) * (uint32_t)c.K * 4u;
#pragma unroll
    for (int i = 0; i < LOADS_B; ++i) ln.b[i] = b0 + (uint32_t)(i * 8) * (uint32_t)c.N * 4u;
    return ln;
  }
  // The scalar parts of the loads of stage t into ring slot `slot`, formed
  // once per stage: this wave's 1 KiB piece of the slot (LDS; wave_lds is
  // the piece in slot 0) and the byte offsets of k-stage t in A (along a
  // row) and B (down the rows).
  struct Dst {
    uint32_t lds, ka, kb;
  };
  // Materialises a stage's load descriptors in scalar registers at this
  // point of the program (nothing moves their computation later). They are
  // uniform by construction; readfirstlane only tells the compiler so.
  static __device__ __forceinline__ void pin(Dst& d) {
    d.lds = __builtin_amdgcn_readfirstlane(d.lds);
    d.ka = __builtin_amdgcn_readfirstlane(d.ka);
    d.kb = __builtin_amdgcn_readfirstlane(d.kb);
    asm volatile("" : "+s"(d.lds), "+s"(d.ka), "+s"(d.kb));
  }
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

  // Operands of k-group g (8 k values): one 16-byte A read per 32-row
  // block (the quad 2g+h of the lane's row), four B dwords per 32-column
  // block.
  struct Frag {
    f32x4 a4[2];
    float bv[2][4];
  };
  static __device__ __forceinline__ void load_frag(const char* abase, int g, Frag& f) {
    const int w = threadIdx.x >> 6, l = lane_id();
    const int wm = w & 1, wn = w >> 1;
    const int lr = l & 31, h = l >> 5;
    const float* bbase = (const float*)(abase + A_STAGE);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int row = wm * 64 + rb * 32 + lr;
      const int q = (2 * g + h) ^ aswz(row);
      f.a4[rb] = *(const f32x4*)(abase + row * 128 + q * 16);
    }
    // Row k = 8g + 4h + s has bswz(k) = h << 3 for every s.
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int col = wn * 64 + cb * 32 + lr;
      const int cpos = (((col >> 2) ^ (h << 3)) << 2) | (col & 3);
#pragma unroll
      for (int s = 0; s < 4; ++s) f.bv[cb][s] = bbase[(8 * g + 4 * h + s) * TN + cpos];
    }
  }

  // NST consecutive k-stages of MFMAs out of ring slots slot .. slot+NST-1
  // (contiguous in LDS), as one sequence of k-groups in ascending k. The
  // operands of group g+1 are read from LDS while group g's 16 MFMAs run.
  // `pre` runs after the first group's operand reads are issued (the
  // preempt-flag check: its LDS read overlaps theirs); if it returns false
  // the stages are abandoned before any accumulator changes and the call
  // returns false. `mid(i)`, i = 0..NST*LOADS-1, runs after MFMA 2i+1 of the
  // first groups (8 per group): the stage loops issue the next stages'
  // direct-to-LDS load i there, under the matrix work.
  template <int NST, class Pre, class Mid>
  static __device__ __forceinline__ bool compute_n(const char* ring, int slot, Acc& acc,
                                                   Pre&& pre, Mid&& mid) {
    const char* abase = ring + slot * STAGE;
    constexpr int GS = KS / 8;    // k-groups per stage
    constexpr int GG = GS * NST;  // k-groups in all
    Frag f[2];
    load_frag(abase, 0, f[0]);
    if (!pre()) return false;
#pragma unroll
    for (int g = 0; g < GG; ++g) {
      // The reads of group g+1 are issued ahead of group g's 16 MFMAs (the
      // scheduling barrier keeps the compiler from sinking each read next to
      // its first use, where the LDS latency would stall the matrix pipe).
      if (g + 1 < GG) load_frag(abase + ((g + 1) / GS) * STAGE, (g + 1) % GS, f[(g + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      const Frag& c = f[g & 1];
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const int s = m >> 2, rb = (m >> 1) & 1, cb = m & 1;
        acc.c[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x2f32(c.a4[rb][s], c.bv[cb][s],
                                                             acc.c[rb][cb], 0, 0, 0);
        if ((m & 1) && g * 8 + (m >> 1) < NST * LOADS) {
          __builtin_amdgcn_sched_barrier(0);
          mid(g * 8 + (m >> 1));
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    return true;
  }
  // The ring's stage group (GROUP stages).
  template <class Pre, class Mid>
  static __device__ __forceinline__ bool compute(const char* ring, int slot, Acc& acc,
                                                 Pre&& pre, Mid&& mid) {
    return compute_n<GROUP>(ring, slot, acc, static_cast<Pre&&>(pre), static_cast<Mid&&>(mid));
  }
  static __device__ __forceinline__ void compute(const char* ring, int slot, Acc& acc) {
    compute(ring, slot, acc, [] { return true; }, [](int) {});
  }

  // Output element (tile-relative row, col) of accumulator register e.
  static __device__ __forceinline__ void coord(int e, int& r, int& c) {
    const int w = threadIdx.x >> 6, l = lane_id();
    const int wm = w & 1, wn = w >> 1, rb = e >> 5, cb = (e >> 4) & 1, q = e & 15;
    r = wm * 64 + rb * 32 + 8 * (q >> 2) + 4 * (l >> 5) + (q & 3);
    c = wn * 64 + cb * 32 + (l & 31);
  }
  static __device__ __forceinline__ float get(const Acc& a, int e) {
    return a.c[e >> 5][(e >> 4) & 1][e & 15];
  }
  static __device__ __forceinline__ void set(Acc& a, int e, float v) {
    a.c[e >> 5][(e >> 4) & 1][e & 15] = v;
  }

  // Write the accumulators into LDS as the row-major TM x TN tile (the ring
  // is free once a tile's last stage has been computed).
  static __device__ __forceinline__ int pass_row(int, int rr) { return rr; }
  static __device__ __forceinline__ void stage_pass(const Acc& acc, char* lds, int) {
    const int w = threadIdx.x >> 6, l = lane_id();
    const int wm = w & 1, wn = w >> 1;
    const int lr = l & 31, h = l >> 5;
    float* t = (float*)lds;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = wm * 64 + rb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          t[row * TN + wn * 64 + cb * 32 + lr] = acc.c[rb][cb][r];
        }
  }
};

using EngMfma128 = EngMfma128T<1>;
using EngMfma128Pairs = EngMfma128T<2>;

}  // namespace apk
