// engine_bf16x128.hpp -- the bf16 tiles for 2 and 4 blocks per CU: output
// tiles of a bf16 GEMM with fp32 accumulation on the gfx950 matrix cores
// (v_mfma_f32_32x32x16_bf16), sized for the occupancy points at which the
// 256x256 tile cannot run (its fp32 accumulator is half of a CU's register
// file and its ring 128 KiB of the 160 KiB LDS):
//  EngBf16x128     (engine bf16x128, 4 blocks per CU): a 128x128 tile on ONE
//                  wave. The wave owns all 4x4 32x32 accumulators (256 fp32
//                  per lane, in AGPRs) and reads 8 operand fragments per 16
//                  MFMAs; with one wave per block every block barrier folds
//                  away (the compiler drops s_barrier for a one-wave
//                  workgroup), so a block never waits for another wave.
//  EngBf16x256x128 (engine bf16x256x128, 2 blocks per CU): a 256x128 tile on
//                  4 waves (2x2, each 128x64: 128 fp32 per lane), two waves
//                  per SIMD at 2 blocks per CU. Against 128x128 it loads 25%
//                  fewer operand bytes per FLOP (85 instead of 64 FLOP per
//                  byte of A and Bt).
//
// Operands as for the 256x256 engine: A is M x K row-major bf16, B is passed
// transposed (Bt = N x K row-major bf16, C = A . Bt^T), both k-contiguous in
// memory, LDS and operand registers. C is M x N row-major fp32.
//
// Stages and loads. The stage loops see 16-deep k-stages in a 4-slot ring
// taken in pairs (GROUP = 2, one barrier per pair; polls and checkpoints at
// pair boundaries). Memory sees 32-deep load regions: a pair of stages is
// loaded as ONE region of 64-byte rows (32 k of every A row of the tile,
// then of every Bt row), so each row costs one full 64-byte request -- with
// 32-byte rows per stage (one 16-deep stage loaded alone) every request was
// half used, and the L1 hit rate of the 4-block configuration fell to 10%.
// Ring slots 2h and 2h+1 are the two halves of region h (the A half and the
// Bt half); a checkpoint always saves and restores them together (a pair
// site's live stages are the pair). Tiles need an even number of stages:
// K a multiple of 32 (K_ALIGN).
//
// LDS layout (both operands): row r of a region is four 16-byte chunks;
// chunk q is stored at slot q ^ swz(r), swz(r) = (r >> 2) & 3 (the 256x256
// engine's layout, measured conflict-free for these operand reads).
//
// k order: the MFMA k-steps of 16 in ascending k; every output's sum is
// formed in the same order whatever worker computes it and however often it
// is checkpointed and resumed.
//
// Epilogue: the fp32 tile is staged through LDS one accumulator row block of
// every wave per pass (32 rows per wave row), row stride TN + 4 floats.
#pragma once
#include "device.hpp"

namespace apk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int TM_, int THREADS_, int BPC_>
struct EngBf16SmallT {
  static_assert(TM_ == 128 || TM_ == 256, "128 or 256 tile rows");
  static_assert(THREADS_ == 64 || THREADS_ == 256, "1 or 4 waves");
  static constexpr int TM = TM_, TN = 128, KS = 16, NS = 4, GROUP = 2, THREADS = THREADS_;
  static constexpr int WAVES = THREADS / 64;
  // Waves WM x WN over the tile; wave (wm, wn) owns a WTM x WTN sub-tile of
  // RB x CB 32x32 accumulators.
  static constexpr int WM = WAVES == 1 ? 1 : 2, WN = WAVES / WM;
  static constexpr int WTM = TM / WM, WTN = TN / WN, RB = WTM / 32, CB = WTN / 32;
  static constexpr int MFMAS = RB * CB;                     // per k-step per wave
  static constexpr int ACC_PER_THREAD = MFMAS * 16;         // floats
  // Blocks per CU the tile is built for; a wave's registers are 512 / waves
  // per SIMD.
  static constexpr int BLOCKS_PER_CU = BPC_;
  static constexpr int WAVES_PER_SIMD = (BLOCKS_PER_CU * WAVES + 3) / 4;
  static constexpr int MIN_WAVES_PER_SIMD = WAVES_PER_SIMD;
  static constexpr int ELEM_BYTES = 2;                      // bf16 operands
  static constexpr int K_ALIGN = 32;                        // an even number of stages
  static constexpr int ROW_BYTES = 64, CHUNKS = 4;          // region rows: 32 k
  static constexpr int A_REGION = TM * ROW_BYTES;           // 8 / 16 KiB
  static constexpr int REGION = A_REGION + TN * ROW_BYTES;  // 16 / 24 KiB
  static constexpr int STAGE = REGION / 2;                  // a ring slot: half a region
  // offset of the Bt rows in a region (the test hook that corrupts an
  // urgent tile's staged B adds to the float there)
  static constexpr int A_STAGE = A_REGION;
  static constexpr int RLOADS = REGION / (THREADS * 16);    // loads per region
  static constexpr int RLOADS_A = A_REGION / (THREADS * 16);
  static constexpr int LOADS = RLOADS / 2;                  // per stage
  static constexpr int ROWS_PER_WAVE = 64 / CHUNKS;         // rows of one wave's load
  // Epilogue: one accumulator row block of every wave per pass.
  static constexpr int STORE_PASSES = RB, PASS_ROWS = 32 * WM, STAGE_LD = TN + 4;
  static constexpr int RING_BYTES = NS * STAGE;             // 32 / 48 KiB
  static constexpr int EPI_BYTES = PASS_ROWS * STAGE_LD * 4;
  static constexpr int LDS_BYTES = RING_BYTES > EPI_BYTES ? RING_BYTES : EPI_BYTES;

  struct Acc {
    f32x16 c[RB][CB];
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
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) a.c[i][j][r] = 0.0f;
  }

  static __device__ __forceinline__ int swz(int r) { return (r >> 2) & 3; }

  // Direct-to-LDS loads of one region: load i fills rows
  // ROWS_PER_WAVE * (WAVES * i + wave) + lane / CHUNKS of the A rows (i <
  // RLOADS_A) or of the Bt rows; lane l writes slot l % CHUNKS of its row, so
  // it reads the row's chunk (l % CHUNKS) ^ swz(row) from memory. The
  // swizzle uses only row bits that i does not change, so each lane's offset
  // of load i is fixed per tile (one register per load); a region only adds
  // the scalar k offset.
  struct Lane {
    uint32_t a[RLOADS_A], b[RLOADS - RLOADS_A];
  };
  static __device__ __forceinline__ Lane lane_offsets(const Ctx& c, int row0, int col0) {
    const int w = wave_id(), l = lane_id();
    const int r = w * ROWS_PER_WAVE + l / CHUNKS;
    const int q = (l % CHUNKS) ^ swz(r);
    const uint32_t a0 = (uint32_t)(((row0 + r) * c.K + 8 * q) * 2);
    const uint32_t b0 = (uint32_t)(((col0 + r) * c.K + 8 * q) * 2);
    Lane ln;
#pragma unroll
    for (int i = 0; i < RLOADS_A; ++i)
      ln.a[i] = a0 + (uint32_t)(i * WAVES * ROWS_PER_WAVE) * (uint32_t)c.K * 2u;
#pragma unroll
    for (int i = 0; i < RLOADS - RLOADS_A; ++i)
      ln.b[i] = b0 + (uint32_t)(i * WAVES * ROWS_PER_WAVE) * (uint32_t)c.K * 2u;
    return ln;
  }
  // Scalar parts of the loads of stage t into ring slot `slot`: this wave's
  // piece of the slot's region (LDS), the byte offset of the region along a
  // row, and the operand resources. Only the first stage of a pair (t even)
  // carries the region's loads; k = NO_LOADS marks the second. A region past
  // the tile's end (t >= S) is read through resources of zero length: every
  // lane reads zeros and no memory is touched.
  struct Dst {
    uint32_t lds, k;
    i32x4 ra, rb;
  };
  static constexpr uint32_t NO_LOADS = 0xffffffffu;
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
    const uint32_t k = (t & 1) ? NO_LOADS : (uint32_t)((real ? t : 0) * KS * 2);
    return Dst{wave_lds + (uint32_t)((slot & ~1) * STAGE), k, real ? c.ra : za,
               real ? c.rb : zb};
  }
  // Byte offset inside a region of region load i's piece (thread t's 16
  // bytes of load i land at region + region_off(i) + 16 t).
  static constexpr uint32_t region_off(int i) {
    return (uint32_t)(i < RLOADS_A ? i * WAVES * 1024
                                   : A_REGION + (i - RLOADS_A) * WAVES * 1024);
  }
  // Thread t's 16 bytes of the last load of the pair whose second stage is
  // in ring slot sl (odd) are at slot sl + dma_lds_off(LOADS - 1) + 16 t.
  static constexpr uint32_t dma_lds_off(int i) { return region_off(RLOADS / 2 + i) - STAGE; }
  static __device__ __forceinline__ void region_load(const Lane& ln, const Dst& d, int i) {
    if (i < RLOADS_A)
      dma_x4(d.ra, d.lds, region_off(i), ln.a[i], d.k);
    else
      dma_x4(d.rb, d.lds, region_off(i), ln.b[i - RLOADS_A], d.k);
  }
  // Load i of stage d alone (prologues and restarts): the first stage of a
  // pair issues the pair's region (two loads per i), the second nothing.
  static __device__ __forceinline__ void issue_one(const Ctx&, const Lane& ln, const Dst& d,
                                                   int i) {
    if (d.k != NO_LOADS) {
      region_load(ln, d, 2 * i);
      region_load(ln, d, 2 * i + 1);
    }
  }
  // Load i (< GROUP * LOADS) of a pair: region load i of its first stage.
  static __device__ __forceinline__ void issue_group(const Ctx&, const Lane& ln, const Dst& d0,
                                                     const Dst&, int i) {
    region_load(ln, d0, i);
  }

  // Operands of k-step j (16 k values) of a region: one 16-byte read per
  // 32-row block of A and per 32-column block of Bt; lanes 0-31 take k 0-7
  // of the step, lanes 32-63 k 8-15.
  struct Frag {
    bf16x8 a[RB], b[CB];
  };
  static __device__ __forceinline__ void load_frag(const char* rbase, int j, Frag& f) {
    const int w = threadIdx.x >> 6, l = lane_id();
    const int wm = w % WM, wn = w / WM;
    const int lr = l & 31, q = 2 * j + (l >> 5);
    const char* bbase = rbase + A_REGION;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int row = wm * WTM + rb * 32 + lr;
      f.a[rb] = *(const bf16x8*)(rbase + row * ROW_BYTES + ((q ^ swz(row)) << 4));
    }
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int col = wn * WTN + cb * 32 + lr;
      f.b[cb] = *(const bf16x8*)(bbase + col * ROW_BYTES + ((q ^ swz(col)) << 4));
    }
  }

  // MFMAs of a pair per load of the next pair issued among them (the loads
  // go out over the first GROUP * LOADS * IV MFMAs).
  static constexpr int IV = 2 * MFMAS / (GROUP * LOADS);
  static_assert(IV >= 1 && IV * GROUP * LOADS <= 2 * MFMAS, "loads spread over the MFMAs");

  // One pair: the region in ring slots slot and slot+1, its two k-steps of
  // MFMAS MFMAs per wave in ascending k, the operands of the second read
  // while the first's MFMAs run. `pre` runs first (false abandons the pair
  // before any accumulator changes); `mid(i)`, i = 0..GROUP*LOADS-1, runs
  // after MFMA (i+1)*IV-1 of the pair: the stage loops issue the next pair's
  // load i there.
  template <class Pre, class Mid>
  static __device__ __forceinline__ bool compute(const char* ring, int slot, Acc& acc,
                                                 Pre&& pre, Mid&& mid) {
    const char* rbase = ring + slot * STAGE;
    Frag f[2];
    if (!pre()) return false;
    load_frag(rbase, 0, f[0]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (j == 0) load_frag(rbase, 1, f[1]);
      const Frag& c = f[j];
#pragma unroll
      for (int m = 0; m < MFMAS; ++m) {
        const int rb = m / CB, cb = m % CB;
        acc.c[rb][cb] =
            __builtin_amdgcn_mfma_f32_32x32x16_bf16(c.a[rb], c.b[cb], acc.c[rb][cb], 0, 0, 0);
        const int g = j * MFMAS + m + 1;  // MFMAs of the pair issued so far
        if (g % IV == 0 && g / IV <= GROUP * LOADS) {
          __builtin_amdgcn_sched_barrier(0);
          mid(g / IV - 1);
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
    const int wm = w % WM, wn = w / WM, blk = e >> 4, rb = blk / CB, cb = blk % CB, i = e & 15;
    r = wm * WTM + rb * 32 + 8 * (i >> 2) + 4 * (l >> 5) + (i & 3);
    c = wn * WTN + cb * 32 + (l & 31);
  }
  static __device__ __forceinline__ float get(const Acc& a, int e) {
    return a.c[(e >> 4) / CB][(e >> 4) % CB][e & 15];
  }
  static __device__ __forceinline__ void set(Acc& a, int e, float v) {
    a.c[(e >> 4) / CB][(e >> 4) % CB][e & 15] = v;
  }

  // Epilogue pass p: accumulator row block rb = p of every wave into LDS as
  // rows [wm*32, wm*32+32) of a PASS_ROWS x TN tile; LDS row rr holds tile
  // row pass_row(p, rr).
  static __device__ __forceinline__ void stage_pass(const Acc& acc, char* lds, int p) {
    const int w = threadIdx.x >> 6, l = lane_id();
    const int wm = w % WM, wn = w / WM;
    float* t = (float*)lds;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int rr = wm * 32 + 8 * (i >> 2) + 4 * (l >> 5) + (i & 3);
        t[rr * STAGE_LD + wn * WTN + cb * 32 + (l & 31)] = acc.c[p][cb][i];
      }
  }
  static __device__ __forceinline__ int pass_row(int p, int rr) {
    return (rr >> 5) * WTM + p * 32 + (rr & 31);
  }
};

// 128x128 on one wave, 4 blocks per CU
using EngBf16x128 = EngBf16SmallT<128, 64, 4>;
// 256x128 on four waves, 2 blocks per CU
using EngBf16x256x128 = EngBf16SmallT<256, 256, 2>;

}  // namespace apk
