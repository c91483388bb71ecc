// engine_valu64.hpp -- the reference's 64x64 fp32 SGEMM tile semantics on
// gfx950 vector ALUs: every output is one fmaf chain over k in ascending order
// (reference src/tile.cuh:62-107), so the result is bit-identical to a
// correctly rounded sequential fmaf on the host.
//
// Block: 256 threads = 4 wave64s; thread (tx = t%16, ty = t/16) owns the 4x4
// outputs rows ty*4..+3, cols tx*4..+3 (the reference's mapping).
// Stage: k depth 32. A stage is As[64][33] (one pad float per row keeps the
// per-row column reads on distinct banks), B stage is Bs[32][64] read as
// 16-byte vectors. Global loads for stage s+1 are issued into registers
// before the FMAs of stage s, so load latency overlaps compute.
#pragma once
#include "device.hpp"

namespace apk {

struct EngValu64 {
  static constexpr int TM = 64, TN = 64, KS = 32, THREADS = 256;
  static constexpr int LDS_BYTES = (TM * (KS + 1) + KS * TN) * 4;

  struct Acc {
    float v[4][4];
  };

  struct Ctx {
    const float* A;
    const float* B;
    int K, N;
  };

  static __device__ __forceinline__ Ctx make_ctx(const float* A, const float* B,
                                                 int, int N, int K) {
    Ctx c;
    c.A = A;
    c.B = B;
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

  struct Regs {
    float4 a[2], b[2];
  };

  static __device__ __forceinline__ void fetch(const Ctx& c, int row0, int col0,
                                               int s, Regs& r) {
    const int t = threadIdx.x, k0 = s * KS;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = t + i * THREADS;  // 512 float4 per operand stage
      const int ar = idx >> 3, aq = idx & 7;
      r.a[i] = *(const float4*)(c.A + (size_t)(row0 + ar) * c.K + k0 + 4 * aq);
      const int br = idx >> 4, bq = idx & 15;
      r.b[i] = *(const float4*)(c.B + (size_t)(k0 + br) * c.N + col0 + 4 * bq);
    }
  }

  static __device__ __forceinline__ void put(char* smem, const Regs& r) {
    float* As = (float*)smem;            // [64][33]
    float* Bs = As + TM * (KS + 1);      // [32][64]
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = t + i * THREADS;
      const int ar = idx >> 3, aq = idx & 7;
      float* ap = As + ar * (KS + 1) + 4 * aq;
      ap[0] = r.a[i].x;
      ap[1] = r.a[i].y;
      ap[2] = r.a[i].z;
      ap[3] = r.a[i].w;
      const int br = idx >> 4, bq = idx & 15;
      *(float4*)(Bs + br * TN + 4 * bq) = r.b[i];
    }
  }

  static __device__ __forceinline__ void compute(const char* smem, Acc& acc) {
    const float* As = (const float*)smem;
    const float* Bs = As + TM * (KS + 1);
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      float a[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[(ty * 4 + i) * (KS + 1) + kk];
      const float4 b = *(const float4*)(Bs + kk * TN + tx * 4);
      const float bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc.v[i][j] = fmaf(a[i], bb[j], acc.v[i][j]);
    }
  }

  template <class Hook>
  static __device__ __forceinline__ void mainloop(char* smem, const Ctx& c,
                                                  Acc& acc, int row0, int col0,
                                                  int s_begin, int s_end,
                                                  Hook&& hook) {
    Regs r;
    if (s_begin < s_end) fetch(c, row0, col0, s_begin, r);
    for (int s = s_begin; s < s_end; ++s) {
      hook(s);
      put(smem, r);
      __syncthreads();
      if (s + 1 < s_end) fetch(c, row0, col0, s + 1, r);
      compute(smem, acc);
      __syncthreads();
    }
  }

  static __device__ __forceinline__ void store(const Acc& acc, float* C, int N,
                                               int row0, int col0) {
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 v = {acc.v[i][0], acc.v[i][1], acc.v[i][2], acc.v[i][3]};
      *(float4*)(C + (size_t)(row0 + ty * 4 + i) * N + col0 + tx * 4) = v;
    }
  }
};

}  // namespace apk
