// engine_bf16x256.hpp -- 256x256 output tile of a bf16 GEMM with fp32
// accumulation on the gfx950 matrix cores (v_mfma_f32_32x32x16_bf16), fed by
// a 4-slot LDS ring of buffer_load_dwordx4 ... lds (direct-to-LDS) that is
// synchronised once per pair of k-stages.
//
// Operands: A is M x K row-major bf16; B is passed transposed, Bt = N x K
// row-major bf16 (C = A . Bt^T), so that both operands are k-contiguous in
// memory, in LDS and in the MFMA operand registers (8 consecutive k per lane
// = one 16-byte LDS read). C is M x N row-major fp32.
//
// Block: 512 threads = 8 wave64s in a 2x4 arrangement, two per SIMD; each
// wave owns a 128x64 sub-tile held as 4x2 32x32 accumulators (128 fp32 per
// lane). A wave then needs ~200 of the SIMD's 512 registers per lane instead
// of all 512: the preemptible kernel runs without spilling, and a small
// kernel on another stream (the flag raise of the retreat arm) still finds
// registers on every CU.
// Stage: k depth KS=32 -> A stage 256 rows x 64 B (16 KiB) + Bt stage 256
// rows x 64 B (16 KiB); 4 slots = 128 KiB of the 160 KiB LDS (1 block/CU).
// A k-stage is only 16 MFMAs per wave (1024 matrix-pipe cycles per SIMD),
// and every barrier costs a fixed ~560 cycles per SIMD (all waves arrive,
// then wait for their first operands): the stage loops therefore take the
// stages in pairs (GROUP = 2), one barrier per pair, with the next pair's
// loads issued under the current pair's first stage. A tile of odd length
// ends with a pair whose second stage is all zeros.
//
// LDS layout (both operands): row r of a stage is 64 B = four 16-byte
// chunks; chunk q is stored at slot q ^ swz(r), swz(r) = (r >> 2) & 3. A
// 32-row operand read (lanes 0-31 chunk 2j, lanes 32-63 chunk 2j+1) then
// takes the minimum 4 LDS cycles per ds_read_b128 on gfx950: measured with
// SQ_LDS_BANK_CONFLICT on a probe of this exact access pattern, where
// ((r >> 1) ^ (r >> 3)) & 3 and (r >> 1) & 3 cost 8 cycles (2-way) and r & 3
// costs 16; (r >> 2) & 3, (r >> 3) & 3, (r ^ (r >> 2)) & 3 and
// ((r >> 1) ^ (r >> 2)) & 3 are conflict-free.
//
// k order: a k-stage is two MFMA k-steps of 16, in ascending k; every
// output's sum is formed in the same order whatever worker computes it and
// however often it is checkpointed and resumed.
//
// Epilogue: the fp32 tile (256 KiB) does not fit the 128 KiB ring, so it is
// staged in 4 passes of 64 rows (32 rows of each wave row): the waves write
// one 32x32 accumulator row block each into LDS, then the whole block moves
// the 64 rows to C with 16-byte coalesced stores (and fingerprints them).
#pragma once
#include "device.hpp"

namespace apk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

struct EngBf16x256 {
  static constexpr int TM = 256, TN = 256, KS = 32, NS = 4, GROUP = 2, THREADS = 512;
  // Waves per SIMD at most (1 block of 8 waves per CU): the register budget the
  // compiler may schedule for.
  static constexpr int WAVES_PER_SIMD = 2;
  static constexpr int MIN_WAVES_PER_SIMD = 1;  // occupancy the registers must allow
  static constexpr int ROW_BYTES = KS * 2;                  // 64 B
  static constexpr int A_STAGE = TM * ROW_BYTES;            // 16 KiB
  static constexpr int B_STAGE = TN * ROW_BYTES;            // 16 KiB
  static constexpr int STAGE = A_STAGE + B_STAGE;           // 32 KiB
  static constexpr int LDS_BYTES = NS * STAGE;              // 128 KiB
  static constexpr int LOADS_A = A_STAGE / (THREADS * 16);  // 2 per thread
  static constexpr int LOADS_B = B_STAGE / (THREADS * 16);  // 2 per thread
  static constexpr int LOADS = LOADS_A + LOADS_B;
  static constexpr int WAVES = THREADS / 64;
  static constexpr int ACC_PER_THREAD = 128;                // floats
  static constexpr int ELEM_BYTES = 2;                      // bf16 operands
  // Epilogue staging: STORE_PASSES passes of PASS_ROWS tile rows through LDS,
  // row stride STAGE_LD floats (4 floats of padding: the two half-waves write
  // rows 4 apart, which then fall on different banks).
  static constexpr int STORE_PASSES = 4, PASS_ROWS = 64, STAGE_LD = TN + 4;

  struct Acc {
    f32x16 c[4][2];
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
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) a.c[i][j][r] = 0.0f;
  }

  static __device__ __forceinline__ int swz(int r) { return (r >> 2) & 3; }

  // Direct-to-LDS loads of one k-stage: load i (0..LOADS-1) fills the
  // 1 KiB piece i*8 + wave of the A stage (i < 2) or of the Bt stage, i.e.
  // 16 rows, row 128*i + 16*wave + lane/4, chunk slot lane%4. The swizzle of
  // a row uses only its bits 2-3, so each lane's offset of load i is fixed
  // per tile (Lane, one register per load) and stage s only adds scalar
  // offsets.
  struct Lane {
    uint32_t a[LOADS_A], b[LOADS_B];
  };
  static __device__ __forceinline__ Lane lane_offsets(const Ctx& c, int row0, int col0) {
    const int w = wave_id(), l = lane_id();
    const int r = w * 16 + (l >> 2);
    const int q = (l & 3) ^ swz(r);
    const uint32_t a0 = (uint32_t)(((row0 + r) * c.K + 8 * q) * 2);
    const uint32_t b0 = (uint32_t)(((col0 + r) * c.K + 8 * q) * 2);
    Lane ln;
#pragma unroll
    for (int i = 0; i < LOADS_A; ++i) ln.a[i] = a0 + (uint32_t)(i * WAVES * 16) * (uint32_t)c.K * 2u;
#pragma unroll
    for (int i = 0; i < LOADS_B; ++i) ln.b[i] = b0 + (uint32_t)(i * WAVES * 16) * (uint32_t)c.K * 2u;
    return ln;
  }
  // The scalar parts of the loads of stage t into ring slot `slot`, formed
  // once per stage: this wave's 1 KiB piece of the slot (LDS; wave_lds is
  // the piece in slot 0), the byte offset of k-stage t along a row, and the
  // operand resources. A stage past the tile's end (t >= S) is read through
  // resources of zero length: every lane reads zeros and no memory is
  // touched, so the slot holds a stage of zeros (the second stage of a last
  // pair of an odd-length tile is computed on it and adds nothing).
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
  // Byte offset inside a ring slot of load i's piece: thread t's 16 bytes of
  // load i land at slot + dma_lds_off(i) + 16 t.
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

  // Operands of k-step j (16 k values): one 16-byte read per 32-row block of
  // A and per 32-column block of Bt.
  struct Frag {
    bf16x8 a[4], b[2];
  };
  static __device__ __forceinline__ void load_frag(const char* abase, int j, Frag& f) {
    const int w = threadIdx.x >> 6, l = lane_id();
    const int wm = w & 1, wn = w >> 1;
    const int lr = l & 31, q = 2 * j + (l >> 5);
    const char* bbase = abase + A_STAGE;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const int row = wm * 128 + rb * 32 + lr;
      f.a[rb] = *(const bf16x8*)(abase + row * ROW_BYTES + ((q ^ swz(row)) << 4));
    }
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int col = wn * 64 + cb * 32 + lr;
      f.b[cb] = *(const bf16x8*)(bbase + col * ROW_BYTES + ((q ^ swz(col)) << 4));
    }
  }

  static constexpr int J = KS / 16;  // MFMA k-steps per stage

  // One group: the GROUP = 2 k-stages in ring slots slot and slot+1 (one
  // half of the ring, contiguous in LDS), as one sequence of 2*J MFMA
  // k-steps in ascending k, the operands of k-step j+1 read while k-step j's
  // MFMAs run -- across the stage boundary too. `pre` runs first (returning
  // false abandons the group before any accumulator changes); `mid(i)`,
  // i = 0..GROUP*LOADS-1, runs after MFMA 2i+1 of the group (k-step i/4,
  // MFMA 2(i%4)+1): the stage loops issue the next group's direct-to-LDS
  // load i there, one per two MFMAs.
  template <class Pre, class Mid>
  static __device__ __forceinline__ bool compute(const char* ring, int slot, Acc& acc,
                                                 Pre&& pre, Mid&& mid) {
    const char* gbase = ring + slot * STAGE;
    constexpr int JG = J * GROUP;
    Frag f[2];
    // pre() runs before any operand is in registers: a yield inside it
    // (checkpoint, urgent tiles, restore) then needs only the accumulators
    // live, which keeps the kernel within the register file.
    if (!pre()) return false;
    load_frag(gbase, 0, f[0]);
#pragma unroll
    for (int j = 0; j < JG; ++j) {
      if (j + 1 < JG) load_frag(gbase + ((j + 1) / J) * STAGE, (j + 1) % J, f[(j + 1) & 1]);
      const Frag& c = f[j & 1];
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int rb = m >> 1, cb = m & 1;
        acc.c[rb][cb] =
            __builtin_amdgcn_mfma_f32_32x32x16_bf16(c.a[rb], c.b[cb], acc.c[rb][cb], 0, 0, 0);
        if ((m & 1) && j * 4 + (m >> 1) < GROUP * LOADS) {
          __builtin_amdgcn_sched_barrier(0);
          mid(j * 4 + (m >> 1));
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
    r = wm * 128 + rb * 32 + 8 * (i >> 2) + 4 * (l >> 5) + (i & 3);
    c = wn * 64 + cb * 32 + (l & 31);
  }
  static __device__ __forceinline__ float get(const Acc& a, int e) {
    return a.c[e >> 5][(e >> 4) & 1][e & 15];
  }
  static __device__ __forceinline__ void set(Acc& a, int e, float v) {
    a.c[e >> 5][(e >> 4) & 1][e & 15] = v;
  }

  // Epilogue pass p: accumulator row block rb = p of every wave into LDS as
  // rows [wm*32, wm*32+32) of a PASS_ROWS x TN tile (row stride STAGE_LD);
  // LDS row rr holds tile row pass_row(p, rr).
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
    return (rr >> 5) * 128 + p * 32 + (rr & 31);
  }
};

}  // namespace apk
