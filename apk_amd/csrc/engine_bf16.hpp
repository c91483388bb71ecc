// engine_bf16.hpp -- the bf16 GEMM tiles: output tiles of C = A . Bt^T with
// bf16 operands and fp32 accumulation on the gfx950 matrix cores
// (v_mfma_f32_32x32x16_bf16), fed by a 4-slot LDS ring of
// buffer_load_dwordx4 ... lds (direct-to-LDS) that is synchronised once per
// pair of k-stages. One template, three tiles:
//  EngBf16x256     (engine bf16x256, 1 block per CU): 256x256 on 8 waves
//                  (2x4, each 128x64: 128 fp32 per lane), two waves per SIMD;
//                  a 256 KiB fp32 accumulator is half of a CU's register
//                  file, so no second block fits. A wave of the poll-off and
//                  retreat kernels takes at most 248 of its SIMD's 256
//                  registers per lane (allocated in 8s), so a small kernel
//                  launched on another stream while the grid runs (the
//                  retreat arm's flag raise, the clock probes) still finds
//                  registers on every SIMD; the cooperative chunk-, stage-
//                  and issue-site kernels, whose generations come from the
//                  grid's own setter, take 250-255. Its pairs are
//                  software-pipelined across the barrier (compute_pl). (The same tile on 4 waves of 128x128 is
//                  no faster, and its polled kernels take all 512 registers
//                  of each SIMD: the flag-raise kernel then waits for the
//                  job to end.)
//  EngBf16x128     (engine bf16x128, 4 blocks per CU): 128x128 on ONE wave
//                  (all 4x4 32x32 accumulators, 256 fp32 per lane, in AGPRs;
//                  8 operand reads per 16 MFMAs). With one wave per block
//                  every block barrier folds away (the compiler drops
//                  s_barrier for a one-wave workgroup). At 4 blocks per CU
//                  its polled kernels fill every SIMD's registers, so it
//                  serves the cooperative arm (device-raised generations);
//                  the retreat arm needs a grid that leaves room in every
//                  dispatch domain.
//  EngBf16x256x128 (engine bf16x256x128, 2 blocks per CU): 256x128 on 4 waves
//                  (2x2, each 128x64), two waves per SIMD; 25% fewer operand
//                  bytes per FLOP than 128x128 (85 instead of 64 FLOP per
//                  byte of A and Bt).
//
// Operands: A is M x K row-major bf16; B is passed transposed, Bt = N x K
// row-major bf16, so that both operands are k-contiguous in memory, in LDS
// and in the MFMA operand registers (8 consecutive k per lane = one 16-byte
// LDS read). C is M x N row-major fp32.
//
// Stages, pairs and load regions. The stage loops see KS-deep k-stages in a
// 4-slot ring taken in pairs (GROUP = 2): one barrier per pair, the next
// pair's loads issued under the current pair's MFMAs, polls and checkpoints
// at pair boundaries. Memory sees load REGIONS: a pair's two stages are
// loaded as one region of 2 KS k -- all TM rows of A, then all TN rows of Bt,
// each row 4 KS bytes -- by one set of loads. Loading each stage alone gives
// rows half as long: the small tiles' 16-deep stages used half of each
// 64-byte request (the 4-block configuration's L1 hit rate fell to 10% and
// its L2 requests doubled), and the 256x256 tile's 32-deep stages half of
// each 128-byte line. Ring slots 2h and 2h+1 are the two halves of region h
// (A half, Bt half); a checkpoint always saves and restores them together (a
// pair site's live stages are the pair), and tiles need an even number of
// stages (K_ALIGN = 2 KS).
//
// LDS layout (both operands): row r of a region is CHUNKS 16-byte chunks;
// chunk q is stored at slot q ^ swz(r). 64-byte rows: swz(r) = (r >> 2) & 3.
// A 32-row operand read (lanes 0-31 chunk 2j, lanes 32-63 chunk 2j+1) then
// takes the minimum 4 LDS cycles per ds_read_b128 on gfx950: measured with
// SQ_LDS_BANK_CONFLICT on a probe of this exact access pattern, where
// ((r >> 1) ^ (r >> 3)) & 3 and (r >> 1) & 3 cost 8 cycles (2-way) and r & 3
// costs 16; (r >> 2) & 3, (r >> 3) & 3, (r ^ (r >> 2)) & 3 and
// ((r >> 1) ^ (r >> 2)) & 3 are conflict-free. 128-byte rows: swz(r) =
// (r >> 1) & 7, so that 16 consecutive rows reading one chunk fall on 16
// different 16-byte bank groups of the 256-byte bank line (even and odd rows
// on its two halves, eight distinct slots each).
//
// k order: k-steps of 16 in ascending k; every output's sum is formed in the
// same order whatever tile, worker, stage depth or region depth computes it,
// and however often it is checkpointed and resumed: the three tiles give
// bit-identical C.
//
// Epilogue: each wave stores its accumulators straight to C (store_direct:
// one dword store per register = two whole 128-byte row segments). A tile
// that is fingerprinted is instead staged through LDS one accumulator row
// block of every wave per pass (32 rows per wave row), row stride TN + 4
// floats (the two half-waves write rows 4 apart, which then fall on
// different banks), then moved to C with 16-byte coalesced stores and
// hashed.
#pragma once
#include "device.hpp"

namespace apk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int TM_, int TN_, int THREADS_, int BPC_, int KS_, int IVMAX_>
struct EngBf16T {
  static_assert(TM_ == 128 || TM_ == 256, "128 or 256 tile rows");
  static_assert(TN_ == 128 || TN_ == 256, "128 or 256 tile columns");
  static_assert(THREADS_ == 64 || THREADS_ == 256 || THREADS_ == 512, "1, 4 or 8 waves");
  static_assert(KS_ == 16 || KS_ == 32, "16- or 32-deep k-stages");
  static constexpr int TM = TM_, TN = TN_, KS = KS_, NS = 4, GROUP = 2, THREADS = THREADS_;
  static constexpr int WAVES = THREADS / 64;
  // Waves WM x WN over the tile; wave (wm, wn) = (w % WM, w / WM) owns a
  // WTM x WTN sub-tile of RB x CB 32x32 accumulators.
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
  static constexpr int RK = 2 * KS;                         // k per load region
  static constexpr int K_ALIGN = RK;
  static constexpr int ROW_BYTES = RK * 2, CHUNKS = ROW_BYTES / 16;
  static constexpr int A_REGION = TM * ROW_BYTES;
  static constexpr int REGION = A_REGION + TN * ROW_BYTES;
  static constexpr int STAGE = REGION / 2;                  // a ring slot
  // offset of the Bt rows in a region (the test hook that corrupts an
  // urgent tile's staged B adds to the float there)
  static constexpr int A_STAGE = A_REGION;
  static constexpr int RLOADS = REGION / (THREADS * 16);    // loads per region
  static constexpr int RLOADS_A = A_REGION / (THREADS * 16);
  static constexpr int LOADS = RLOADS / 2;                  // per stage
  static constexpr int ROWS_PER_WAVE = 64 / CHUNKS;         // rows of one wave's load
  static_assert(RLOADS_A * THREADS * 16 == A_REGION && RLOADS * THREADS * 16 == REGION,
                "whole loads per operand");
  static_assert(RLOADS % 2 == 0, "a pair's loads split evenly over its stages");
  // Load i of a wave covers rows (WAVES * i + wave) * ROWS_PER_WAVE + ...; the
  // swizzle must not see the WAVES * ROWS_PER_WAVE step (one offset register
  // per load, formed once per tile).
  static_assert((WAVES * ROWS_PER_WAVE) % 16 == 0, "loads keep the swizzle");
  // Epilogue: one accumulator row block of every wave per pass.
  static constexpr int STORE_PASSES = RB, PASS_ROWS = 32 * WM, STAGE_LD = TN + 4;
  static constexpr int RING_BYTES = NS * STAGE;
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

  static __device__ __forceinline__ int swz(int r) {
    return CHUNKS == 4 ? (r >> 2) & 3 : (r >> 1) & 7;
  }

  // Direct-to-LDS loads of one region: load i fills rows
  // ROWS_PER_WAVE * (WAVES * i + wave) + lane / CHUNKS of the A rows (i <
  // RLOADS_A) or of the Bt rows; lane l writes slot l % CHUNKS of its row, so
  // it reads the row's chunk (l % CHUNKS) ^ swz(row) from memory. Each lane's
  // offset of load i is fixed per tile (one register per load); a region only
  // adds the scalar k offset.
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
  // The scalar parts of the loads of stage t into ring slot `slot`, formed
  // once per stage: this wave's 1 KiB piece of the slot's region (LDS), the
  // byte offset of the region along a row, and the operand resources. Only
  // the first stage of a pair (t even) carries the region's loads; k =
  // NO_LOADS marks the second. A region past the tile's end (t >= S) is read
  // through resources of zero length: every lane reads zeros and no memory
  // is touched (the refetch that stands in for the pair after a tile's last).
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
    // only the resources' record counts differ (one select each)
    i32x4 ra = c.ra, rb = c.rb;
    ra.z = real ? c.ra.z : 0;
    rb.z = real ? c.rb.z : 0;
    const uint32_t k = (t & 1) ? NO_LOADS : (uint32_t)((real ? t : 0) * KS * 2);
    return Dst{wave_lds + (uint32_t)((slot & ~1) * STAGE), k, ra, rb};
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

  static constexpr int JG = RK / 16;  // MFMA k-steps per pair (one region)
  // The next pair's loads go out one per IV MFMAs from the pair's start, at
  // most one per IVMAX: issued densely at the front of the pair, they have
  // the rest of it to land. Measured at cfg5 (calibrate, one box): one per
  // MFMA is 2% faster than one per two for the 256x256 tile and 4.6% for
  // the one-wave 128x128 tile; one per two is 2% faster for 256x128.
  static constexpr int IV_FIT = JG * MFMAS / (GROUP * LOADS);
  static constexpr int IV = IV_FIT < IVMAX_ ? IV_FIT : IVMAX_;
  static_assert(IV >= 1, "loads spread over the MFMAs");

  // One pair: the region in ring slots slot and slot+1, MFMAS MFMAs per
  // k-step per wave in ascending k, the operands of k-step j+1 read while
  // k-step j's MFMAs run. `pre` runs first (returning false abandons the pair
  // before any accumulator changes); it runs before any operand is in
  // registers, so a yield inside it (checkpoint, urgent tiles, restore) needs
  // only the accumulators live. `mid(i)`, i = 0..GROUP*LOADS-1, runs after
  // MFMA (i+1)*IV-1 of the pair: the stage loops issue the next pair's load i
  // there.
  template <class Pre, class Mid>
  static __device__ __forceinline__ bool compute(const char* ring, int slot, Acc& acc,
                                                 Pre&& pre, Mid&& mid) {
    const char* gbase = ring + slot * STAGE;
    Frag f[2];
    if (!pre()) return false;
    load_frag(gbase, 0, f[0]);
#pragma unroll
    for (int j = 0; j < JG; ++j) {
      if (j + 1 < JG) load_frag(gbase, j + 1, f[(j + 1) & 1]);
      const Frag& c = f[j & 1];
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

  // The same pair software-pipelined across the barrier: half of its last
  // k-step -- the MFMAs of accumulator rows rb < RT, whose operands (RT A
  // and all CB Bt fragments) are kept in a Tail -- runs in the NEXT pair's
  // call, right after that pair's first operand reads are issued. Those
  // MFMAs (operands already in registers) cover the reads' LDS latency,
  // which otherwise leaves both waves of a SIMD idle after every barrier
  // when both belong to the block that barriered (and the site's flag read
  // with them). With `hasTail` the call first completes the previous pair;
  // without (a job's first pair, or the pair a site stopped at) it skips
  // those MFMAs. Then come the first of the next pair's loads (`mid`, the
  // ones the tail's MFMAs carry), `pre` -- a site's state is that of the
  // stages before this pair, the previous pair included; a pair abandoned
  // there has those loads in flight into the free half of the ring, which a
  // checkpoint drains -- and this pair's k-steps, the rows rb >= RT of its
  // last one included, carrying the other loads. Without `early` those first
  // loads go out right after `pre` instead: a block that may leave at `pre`
  // then has no fresh loads to wait for before it exits. One body for both cases
  // (a uniform branch around the tail's MFMAs): two inlined copies of the
  // pair spilled in the polled kernels. Every accumulator still sees its
  // k-steps in ascending order.
  static constexpr int RT = (RB + 1) / 2;  // accumulator rows whose last k-step is deferred
  struct Tail {
    bf16x8 a[RT], b[CB];
  };
  static constexpr int NT_MF = RT * CB;             // deferred MFMAs
  static constexpr int NH = JG * MFMAS - NT_MF;      // MFMAs of a pair in its own call
  static_assert(NH >= GROUP * LOADS, "a pair without a tail still spreads its loads");
  template <class Pre, class Mid>
  static __device__ __forceinline__ bool compute_pl(const char* ring, int slot, Acc& acc,
                                                    Tail& tail, bool hasTail, bool early,
                                                    Pre&& pre, Mid&& mid) {
    constexpr int NT = NT_MF;  // the previous pair's MFMAs, before `pre`
    constexpr int IV_P = (NT + NH) / (GROUP * LOADS) < IVMAX_ ? (NT + NH) / (GROUP * LOADS)
                                                              : IVMAX_;
    auto hook = [&](int g) {  // after the call's g-th MFMA
      if (g % IV_P == 0 && g / IV_P <= GROUP * LOADS) {
        __builtin_amdgcn_sched_barrier(0);
        mid(g / IV_P - 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    auto mma = [&](const bf16x8& a, const bf16x8& b, int rb, int cb) {
      acc.c[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc.c[rb][cb], 0, 0, 0);
    };
    const char* gbase = ring + slot * STAGE;
    Frag f[2];
    bf16x8 rest[RB - RT];  // the last k-step's A rows RT..RB-1
    load_frag(gbase, 0, f[0]);
    __builtin_amdgcn_sched_barrier(0);
    if (hasTail) {
#pragma unroll
      for (int m = 0; m < NT_MF; ++m) mma(tail.a[m / CB], tail.b[m % CB], m / CB, m % CB);
    }
    // the loads the tail's MFMAs would have carried: before `pre` when
    // `early`, else right after it (a block that may leave at `pre` then has
    // no fresh loads to drain first)
    if (early) {
#pragma unroll
      for (int m = 0; m < NT_MF; ++m) hook(m + 1);
    }
    if (!pre()) return false;
    if (!early) {
#pragma unroll
      for (int m = 0; m < NT_MF; ++m) hook(m + 1);
    }
#pragma unroll
    for (int j = 0; j + 1 < JG; ++j) {
      if (j + 2 < JG) {
        load_frag(gbase, j + 1, f[(j + 1) & 1]);
      } else {
        Frag& last = f[(j + 1) & 1];
        load_frag(gbase, JG - 1, last);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          if (rb < RT) tail.a[rb] = last.a[rb];
          else rest[rb - RT] = last.a[rb];
        }
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) tail.b[cb] = last.b[cb];
      }
      const Frag& c = f[j & 1];
#pragma unroll
      for (int m = 0; m < MFMAS; ++m) {
        mma(c.a[m / CB], c.b[m % CB], m / CB, m % CB);
        hook(NT + j * MFMAS + m + 1);
      }
    }
    // the last k-step's rows RT..RB-1 now; rows 0..RT-1 in the next call
#pragma unroll
    for (int m = 0; m < (RB - RT) * CB; ++m) {
      mma(rest[m / CB], tail.b[m % CB], RT + m / CB, m % CB);
      hook(NT + (JG - 1) * MFMAS + m + 1);
    }
    return true;
  }
  // The last pair's deferred MFMAs, before the accumulators are read.
  static __device__ __forceinline__ void finish_tail(Acc& acc, const Tail& tail) {
#pragma unroll
    for (int m = 0; m < NT_MF; ++m) {
      const int rb = m / CB, cb = m % CB;
      acc.c[rb][cb] =
          __builtin_amdgcn_mfma_f32_32x32x16_bf16(tail.a[rb], tail.b[cb], acc.c[rb][cb], 0, 0, 0);
    }
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

  // The C tile straight from the accumulators, no LDS: accumulator register
  // i of a 32x32 block holds, in lanes 0-31, 32 consecutive columns of one
  // row, and in lanes 32-63 the same columns 4 rows below, so one dword
  // store per register writes two whole 128-byte row segments. Every wave
  // stores its own sub-tile with no barrier. (A fingerprinted tile takes the
  // staged epilogue: its hash, unrolled over every register here, spilled.)
  static __device__ __forceinline__ void store_direct(const Acc& acc, float* C, int ldc,
                                                      int row0, int col0) {
    const int w = threadIdx.x >> 6, l = lane_id();
    const int wm = w % WM, wn = w / WM;
    float* base = C + (size_t)(row0 + wm * WTM + 4 * (l >> 5)) * ldc + col0 + wn * WTN + (l & 31);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float* row = base + (size_t)(rb * 32 + 8 * (i >> 2) + (i & 3)) * ldc;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) row[cb * 32] = acc.c[rb][cb][i];
      }
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

// 256x256 on eight waves, 1 block per CU: 32-deep stages, 64-k regions
using EngBf16x256 = EngBf16T<256, 256, 512, 1, 32, 1>;
// 128x128 on one wave, 4 blocks per CU: 16-deep stages, 32-k regions
using EngBf16x128 = EngBf16T<128, 128, 64, 4, 16, 1>;
// 256x128 on four waves, 2 blocks per CU: 16-deep stages, 32-k regions
using EngBf16x256x128 = EngBf16T<256, 128, 256, 2, 16, 2>;

}  // namespace apk
