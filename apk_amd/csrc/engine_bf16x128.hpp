// engine_bf16x128.hpp -- 128x128 output tile of a bf16 GEMM with fp32
// accumulation on the gfx950 matrix cores (v_mfma_f32_32x32x16_bf16), sized
// so that 2 and 4 blocks share a CU: the occupancy points at which the
// 256x256 tile cannot run (its fp32 accumulator is half of a CU's register
// file and its ring 128 KiB of the 160 KiB LDS).
//
// Operands as for the 256x256 engine: A is M x K row-major bf16, B is passed
// transposed (Bt = N x K row-major bf16, C = A . Bt^T), both k-contiguous in
// memory, LDS and operand registers. C is M x N row-major fp32.
//
// Block: 256 threads = 4 wave64s in a 2x2 arrangement; each wave owns a
// 64x64 sub-tile held as 2x2 32x32 accumulators (64 fp32 per lane). Two
// stage depths (template parameter KS), both with a 4-slot ring taken in
// pairs of stages (GROUP = 2, one barrier per pair, as in the 256x256
// engine):
//  KS = 16 (EngBf16x128, engine bf16x128): one MFMA k-step per stage; A and
//     Bt stages of 128 rows x 32 B, 32 KiB of ring; the LDS block is 33 KiB
//     (the epilogue's staging of 64 padded rows), so 4 blocks take 132 KiB
//     of the CU's 160 KiB, and a wave has 128 registers per lane (4 waves
//     per SIMD).
//  KS = 32 (EngBf16x128K32, engine bf16x128k32): two k-steps per stage, rows
//     of 64 B, 64 KiB of ring: 2 blocks per CU, 256 registers per lane. Twice
//     the MFMAs per barrier: 37-39% faster than KS = 16 at 1 and 2 blocks per
//     CU (8192^3, ABAB), with C bit-identical.
//
// LDS layout (both operands): row r of a stage is KS * 2 bytes = 2 or 4
// 16-byte chunks; chunk q is stored at slot q ^ swz(r), swz(r) = (r >> 3) & 1
// for 32-byte rows and (r >> 2) & 3 for 64-byte rows. A ds_read_b128 is
// served 16 lanes per cycle (256 B); 16 consecutive rows reading one chunk
// then fall on 16 different 16-byte bank groups (the 64-byte layout is the
// 256x256 engine's, measured conflict-free there).
//
// k order: the MFMA k-steps of 16 in ascending k; every output's sum is
// formed in the same order whatever worker computes it, whatever the stage
// depth, and however often it is checkpointed and resumed.
//
// Epilogue: the fp32 tile (64 KiB) is staged in 2 passes of 64 rows (32 rows
// of each wave row), row stride TN + 4 floats.
#pragma once
#include "device.hpp"

namespace apk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int KS_>
struct EngBf16x128T {
  static_assert(KS_ == 16 || KS_ == 32, "16- or 32-deep k-stages");
  static constexpr int TM = 128, TN = 128, KS = KS_, NS = 4, GROUP = 2, THREADS = 256;
  // KS 16: 4 blocks of 4 waves per CU, so every instantiation must fit 128
  // registers per lane; KS 32: 2 blocks (64 KiB ring each), 256 registers.
  static constexpr int WAVES_PER_SIMD = KS == 16 ? 4 : 2;
  static constexpr int MIN_WAVES_PER_SIMD = WAVES_PER_SIMD;
  static constexpr int CHUNKS = KS * 2 / 16;                // 16-byte chunks per row
  static constexpr int ROW_BYTES = KS * 2;                  // 32 / 64 B
  static constexpr int A_STAGE = TM * ROW_BYTES;            // 4 / 8 KiB
  static constexpr int B_STAGE = TN * ROW_BYTES;
  static constexpr int STAGE = A_STAGE + B_STAGE;           // 8 / 16 KiB
  static constexpr int LOADS_A = A_STAGE / (THREADS * 16);  // 1 / 2 per thread
  static constexpr int LOADS_B = B_STAGE / (THREADS * 16);
  static constexpr int LOADS = LOADS_A + LOADS_B;
  static constexpr int WAVES = THREADS / 64;
  static constexpr int ROWS_PER_WAVE = 64 / CHUNKS;         // rows of one wave's load
  static constexpr int ACC_PER_THREAD = 64;                 // floats
  static constexpr int ELEM_BYTES = 2;                      // bf16 operands
  static constexpr int STORE_PASSES = 2, PASS_ROWS = 64, STAGE_LD = TN + 4;
  static constexpr int RING_BYTES = NS * STAGE;             // 32 / 64 KiB
  static constexpr int EPI_BYTES = PASS_ROWS * STAGE_LD * 4;
  static constexpr int LDS_BYTES = RING_BYTES > EPI_BYTES ? RING_BYTES : EPI_BYTES;

  struct Acc {
    f32x16 c[2][2];
  };

  struct Ctx {
    i32x4 ra, rb;
    int K;
  };

  static __device__ __forceinline__ Ctx make_ctx(const void* A, const void* Bt, int M, int N,
                                                 int K) {
    Ctx c;
    c.ra = make_rsrc(A, (uint32_t)((size_t)M * K * 2));
    c.rb = make_rsrc(Bt, (uint32_t)((size_t)N * K * 2));
    c.K = K;
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

  // 32-byte rows: (r >> 3) & 1; 64-byte rows: (r >> 2) & 3 (the 256x256
  // engine's layout).
  static __device__ __forceinline__ int swz(int r) {
    return KS == 16 ? (r >> 3) & 1 : (r >> 2) & 3;
  }

  // Direct-to-LDS loads of one k-stage: load i fills rows
  // ROWS_PER_WAVE * (WAVES * i + wave) + lane / CHUNKS of the A stage (i <
  // LOADS_A) or of the Bt stage; lane l writes slot l % CHUNKS of its row,
  // so it reads the row's chunk (l % CHUNKS) ^ swz(row) from memory. The
  // swizzle uses only row bits that i does not change, so each lane's offset
  // of load i is fixed per tile (one register per load); stage t only adds
  // the scalar k offset.
  struct Lane {
    uint32_t a[LOADS_A], b[LOADS_B];
  };
  static __device__ __forceinline__ Lane lane_offsets(const Ctx& c, int row0, int col0) {
    const int w = wave_id(), l = lane_id();
    const int r = w * ROWS_PER_WAVE + l / CHUNKS;
    const int q = (l % CHUNKS) ^ swz(r);
    const uint32_t a0 = (uint32_t)(((row0 + r) * c.K + 8 * q) * 2);
    const uint32_t b0 = (uint32_t)(((col0 + r) * c.K + 8 * q) * 2);
    Lane ln;
#pragma unroll
    for (int i = 0; i < LOADS_A; ++i)
      ln.a[i] = a0 + (uint32_t)(i * WAVES * ROWS_PER_WAVE) * (uint32_t)c.K * 2u;
#pragma unroll
    for (int i = 0; i < LOADS_B; ++i)
      ln.b[i] = b0 + (uint32_t)(i * WAVES * ROWS_PER_WAVE) * (uint32_t)c.K * 2u;
    return ln;
  }
  // Scalar parts of stage t's loads into ring slot `slot` (as in the 256x256
  // engine): t >= S reads through zero-length resources, i.e. zeros.
  struct Dst {
    uint32_t lds, k;
    i32x4 ra, rb;
  };
  // Materialises a stage's load descriptors in scalar registers at this
  // point of the program (nothing moves their computation later).
  static __device__ __forceinline__ void pin(Dst& d) {
    asm volatile("" : "+s"(d.lds), "+s"(d.k), "+s"(d.ra), "+s"(d.rb));
  }
  static __device__ __forceinline__ Dst stage_dst(uint32_t wave_lds, const Ctx& c, int slot,
                                                  int t, int S) {
    const bool real = t < S;
    i32x4 za = c.ra, zb = c.rb;
    za.z = 0;
    zb.z = 0;
    return Dst{wave_lds + (uint32_t)(slot * STAGE), (uint32_t)((real ? t : 0) * KS * 2),
               real ? c.ra : za, real ? c.rb : zb};
  }
  // Byte offset inside a ring slot of load i's piece (thread t's 16 bytes of
  // load i land at slot + dma_lds_off(i) + 16 t).
  static constexpr uint32_t dma_lds_off(int i) {
    return (uint32_t)(i < LOADS_A ? i * WAVES * 1024 : A_STAGE + (i - LOADS_A) * WAVES * 1024);
  }
  static __device__ __forceinline__ void issue_one(const Ctx&, const Lane& ln, const Dst& d,
                                                   int i) {
    if (i < LOADS_A)
      dma_x4(d.ra, d.lds, dma_lds_off(i), ln.a[i], d.k);
    else
      dma_x4(d.rb, d.lds, dma_lds_off(i), ln.b[i - LOADS_A], d.k);
  }

  // Operands of k-step j (16 k values) of a stage: one 16-byte read per
  // 32-row block of A and per 32-column block of Bt; lanes 0-31 take k 0-7
  // of the step, lanes 32-63 k 8-15.
  struct Frag {
    bf16x8 a[2], b[2];
  };
  static __device__ __forceinline__ void load_frag(const char* sbase, int j, Frag& f) {
    const int w = threadIdx.x >> 6, l = lane_id();
    const int wm = w & 1, wn = w >> 1;
    const int lr = l & 31, q = 2 * j + (l >> 5);
    const char* bbase = sbase + A_STAGE;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int row = wm * 64 + rb * 32 + lr;
      f.a[rb] = *(const bf16x8*)(sbase + row * ROW_BYTES + ((q ^ swz(row)) << 4));
    }
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int col = wn * 64 + cb * 32 + lr;
      f.b[cb] = *(const bf16x8*)(bbase + col * ROW_BYTES + ((q ^ swz(col)) << 4));
    }
  }

  static constexpr int J = KS / 16;  // MFMA k-steps per stage

  // One group: the two k-stages in ring slots slot and slot+1, 4 MFMAs per
  // k-step per wave in ascending k, the operands of k-step j+1 read while
  // k-step j's MFMAs run. `pre` runs first (false abandons the group before
  // any accumulator changes); `mid(i)`, i = 0..GROUP*LOADS-1, runs after
  // MFMA 2i+1: the stage loops issue the next group's load i there.
  template <class Pre, class Mid>
  static __device__ __forceinline__ bool compute(const char* ring, int slot, Acc& acc,
                                                 Pre&& pre, Mid&& mid) {
    const char* gbase = ring + slot * STAGE;
    constexpr int JG = J * GROUP;
    Frag f[2];
    if (!pre()) return false;
    load_frag(gbase, 0, f[0]);
#pragma unroll
    for (int j = 0; j < JG; ++j) {
      if (j + 1 < JG) load_frag(gbase + ((j + 1) / J) * STAGE, (j + 1) % J, f[(j + 1) & 1]);
      const Frag& c = f[j & 1];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int rb = m >> 1, cb = m & 1;
        acc.c[rb][cb] =
            __builtin_amdgcn_mfma_f32_32x32x16_bf16(c.a[rb], c.b[cb], acc.c[rb][cb], 0, 0, 0);
        if ((m & 1) && j * 2 + (m >> 1) < GROUP * LOADS) {
          __builtin_amdgcn_sched_barrier(0);
          mid(j * 2 + (m >> 1));
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    return true;
  }
  static __device__ __forceinline__ void compute(const char* ring, int slot, Acc& acc) {
    compute(ring, slot, acc, [] { return true; }, [](int) {});
  }

  // Output element (tile-relative row, col) of accumulator register e.
  static __device__ __forceinline__ void coord(int e, int& r, int& c) {
    const int w = threadIdx.x >> 6, l = lane_id();
    const int wm = w & 1, wn = w >> 1, rb = e >> 5, cb = (e >> 4) & 1, i = e & 15;
    r = wm * 64 + rb * 32 + 8 * (i >> 2) + 4 * (l >> 5) + (i & 3);
    c = wn * 64 + cb * 32 + (l & 31);
  }
  static __device__ __forceinline__ float get(const Acc& a, int e) {
    return a.c[e >> 5][(e >> 4) & 1][e & 15];
  }
  static __device__ __forceinline__ void set(Acc& a, int e, float v) {
    a.c[e >> 5][(e >> 4) & 1][e & 15] = v;
  }

  // Epilogue pass p: accumulator row block rb = p of every wave into LDS as
  // rows [wm*32, wm*32+32) of a 64 x TN tile; LDS row rr holds tile row
  // pass_row(p, rr).
  static __device__ __forceinline__ void stage_pass(const Acc& acc, char* lds, int p) {
    const int w = threadIdx.x >> 6, l = lane_id();
    const int wm = w & 1, wn = w >> 1;
    float* t = (float*)lds;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int rr = wm * 32 + 8 * (i >> 2) + 4 * (l >> 5) + (i & 3);
        t[rr * STAGE_LD + wn * 64 + cb * 32 + (l & 31)] = acc.c[p][cb][i];
      }
  }
  static __device__ __forceinline__ int pass_row(int p, int rr) {
    return (rr >> 5) * 64 + p * 32 + (rr & 31);
  }
};

using EngBf16x128 = EngBf16x128T<16>;     // 16-deep stages: up to 4 blocks per CU
using EngBf16x128K32 = EngBf16x128T<32>;  // 32-deep stages: up to 2 blocks per CU

}  // namespace apk
