// k_persistent.hip -- the persistent GEMM worker pool (calibration path).
//
// Counterpart of persistent_gemm (reference src/persistent.cu:51-79): a grid
// of resident workers pops output tiles from one fetch-add counter in HBM
// until the tile space is exhausted (termination by queue exhaustion, so
// correctness never depends on co-residency). A tile's K range is walked in
// k_chunk-wide chunks in order; chunk boundaries are the points where the
// preemptible variants poll, and here they are where per-chunk timing
// records are taken.
#include <climits>
#include <mutex>

#include "capi.hpp"
#include "engine_bf16.hpp"
#include "engine_mfma128.hpp"
#include "engine_valu64.hpp"
#include "pipeline.hpp"

namespace apk {

template <class E>
__global__ void __launch_bounds__(E::THREADS) __attribute__((amdgpu_waves_per_eu(E::MIN_WAVES_PER_SIMD, E::WAVES_PER_SIMD)))
    k_persistent_gemm(const void* __restrict__ A, const void* __restrict__ B,
                      float* __restrict__ C, int M, int N, int K, int kChunk,
                      unsigned* next_task, apk_tile_record* log) {
  __shared__ __attribute__((aligned(16))) char ring[E::LDS_BYTES];
  __shared__ unsigned s_task;

  const int tilesN = N / E::TN;
  const unsigned numTasks = (unsigned)((M / E::TM) * tilesN);
  const TaskQueue tq(next_task, M / E::TM, tilesN, numTasks);
  const int home = (int)xcc_id();
  const int nChunks = K / kChunk;
  const int spc = kChunk / E::KS;  // k-stages per chunk
  const typename E::Ctx ctx = E::make_ctx(A, B, M, N, K);
  const uint32_t wl = wave_lds(ring);

  for (;;) {
    // Reconverge before the thread-0 pop (no thread-0 region of the previous
    // iteration may be threaded into this one across the back-edge).
    lds_sync();
    if (threadIdx.x == 0) s_task = tq.pop(home);
    __syncthreads();
    const unsigned task = uniform(s_task);
    __syncthreads();  // every thread has read s_task before it is rewritten
    if (task >= numTasks) break;

    const int row0 = (int)(task / tilesN) * E::TM;
    const int col0 = (int)(task % tilesN) * E::TN;
    int64_t prev = 0;
    apk_tile_record* rec = log ? log + (size_t)task * nChunks : nullptr;

    typename E::Acc acc;
    E::zero(acc);
    // The next stage that opens a chunk record (none when no log is kept):
    // one uniform compare per stage instead of a modulo under a per-thread
    // branch at the top of every stage.
    int nextRec = rec ? 0 : INT_MAX;
    run_stages<E>(ring, wl, ctx, acc, row0, col0, K / E::KS, [&](int s) {
      if (s != nextRec) return;
      nextRec += spc;
      if (threadIdx.x == 0) {
        const int64_t now = wall_ticks();
        const int c = s / spc;
        if (c > 0) {
          rec[c - 1].start = prev;
          rec[c - 1].end = now;
          rec[c - 1].smid = (int)hw_slot();
          rec[c - 1].block = (int)blockIdx.x;
        }
        prev = now;
      }
    });
    store_tile<E>(acc, ring, C, N, row0, col0, false);
    __syncthreads();  // whole tile committed before the clock closes
    if (threadIdx.x == 0 && rec) {
      rec[nChunks - 1].start = prev;
      rec[nChunks - 1].end = wall_ticks();
      rec[nChunks - 1].smid = (int)hw_slot();
      rec[nChunks - 1].block = (int)blockIdx.x;
    }
  }
}

// The urgent job as the reference runs it (urgent_tile, src/urgent_baseline.cu:
// 100-112): one block per output tile, block b computing tile b over the
// whole K, no queue; block 0 stamps the job's start at its first
// instruction and every block raises the job's end once its tile is stored.
template <class E>
__global__ void __launch_bounds__(E::THREADS) __attribute__((amdgpu_waves_per_eu(E::MIN_WAVES_PER_SIMD, E::WAVES_PER_SIMD)))
    k_urgent_tiles(const void* __restrict__ A, const void* __restrict__ B,
                   float* __restrict__ C, int M, int N, int K, long long* start_gt,
                   unsigned long long* end_gt) {
  if (start_gt && blockIdx.x == 0 && threadIdx.x == 0) *start_gt = (long long)wall_ticks();
  __shared__ __attribute__((aligned(16))) char ring[E::LDS_BYTES];
  const int tilesN = N / E::TN;
  const int row0 = (int)(blockIdx.x / (unsigned)tilesN) * E::TM;
  const int col0 = (int)(blockIdx.x % (unsigned)tilesN) * E::TN;
  const typename E::Ctx ctx = E::make_ctx(A, B, M, N, K);
  typename E::Acc acc;
  E::zero(acc);
  run_stages<E>(ring, wave_lds(ring), ctx, acc, row0, col0, K / E::KS, [](int) {});
  store_tile<E>(acc, ring, C, N, row0, col0, false);
  if (end_gt) {
    wait_vmcnt<0>();  // this thread's C stores have completed
    lds_sync();       // ... and every other thread's
    if (threadIdx.x == 0)
      atomic_max_u64(end_gt, (unsigned long long)wall_ticks());
  }
}

template <class E>
static int validate_persistent_gemm(const void* A, const void* B, float* C, int M, int N, int K,
                                    int kChunk, int blocks) {
  APK_REQUIRE(A && B && C, "persistent_gemm: NULL pointer");
  APK_REQUIRE(M > 0 && N > 0 && K > 0, "persistent_gemm: empty shape");
  APK_REQUIRE(M % E::TM == 0 && N % E::TN == 0,
              "persistent_gemm: M=%d N=%d not multiples of the %dx%d tile", M, N,
              E::TM, E::TN);
  APK_REQUIRE(kChunk > 0 && kChunk % E::KS == 0 && K % kChunk == 0,
              "persistent_gemm: k_chunk=%d must divide K=%d and be a multiple "
              "of %d", kChunk, K, E::KS);
  APK_REQUIRE(K % KAlign<E>::value == 0, "persistent_gemm: K=%d must be a multiple of %d", K,
              KAlign<E>::value);
  APK_REQUIRE((size_t)M * K * E::ELEM_BYTES < (1ull << 31) &&
                  (size_t)K * N * E::ELEM_BYTES < (1ull << 31) &&
                  (size_t)M * N < (1ull << 31),
              "persistent_gemm: operands above 2 GiB are not supported");
  APK_REQUIRE(blocks > 0, "persistent_gemm: blocks=%d", blocks);
  return APK_OK;
}

template <class E>
static int launch_persistent_gemm(const void* A, const void* B, float* C,
                                  int M, int N, int K, int kChunk,
                                  unsigned* next, apk_tile_record* log,
                                  int blocks, hipStream_t st) {
  const int rc = validate_persistent_gemm<E>(A, B, C, M, N, K, kChunk, blocks);
  if (rc != APK_OK) return rc;
  APK_REQUIRE(next != nullptr, "persistent_gemm: next_task is NULL");
  hipLaunchKernelGGL(k_persistent_gemm<E>, dim3(blocks), dim3(E::THREADS), 0, st,
                     A, B, C, M, N, K, kChunk, next, log);
  APK_LAUNCHED();
  return APK_OK;
}

// ---------------------------------------------------------------------------
// Allocation-free variant (apk_persistent_gemm_noalloc): the work-queue
// counters live in this file-scope array instead of a caller buffer. In host
// code `scratch` only names the variable; its device address, one per GPU,
// comes from hipGetSymbolAddress on the first call made with that GPU
// current and is the only form in which host code uses it.
static __device__ __align__(256) unsigned scratch[APK_NOALLOC_SCRATCH_WORDS];
static_assert(APK_QUEUE_WORDS <= APK_NOALLOC_SCRATCH_WORDS, "queue counters must fit scratch");

constexpr int kMaxDevices = 64;
static unsigned* g_scratch[kMaxDevices];  // device address of `scratch`, per GPU
static std::mutex g_scratch_mu;

// The counters start every launch at zero. A kernel, not hipMemsetAsync, so
// that the sequence can be captured into a graph and replayed.
__global__ void __launch_bounds__(64) k_zero_words(unsigned* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}

static int scratch_of_current_device(unsigned** out) {
  int dev = -1;
  APK_HIP(hipGetDevice(&dev));
  APK_REQUIRE(dev >= 0 && dev < kMaxDevices, "persistent_gemm_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    APK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    APK_REQUIRE(p != nullptr, "persistent_gemm_noalloc: no device address for scratch");
    g_scratch[dev] = (unsigned*)p;
  }
  *out = g_scratch[dev];
  return APK_OK;
}

template <class E>
static int launch_urgent_tiles(const void* A, const void* B, float* C, int M, int N, int K,
                               long long* start_gt, unsigned long long* end_gt,
                               hipStream_t st) {
  const int rc = validate_persistent_gemm<E>(A, B, C, M, N, K, K, 1);
  if (rc != APK_OK) return rc;
  const int tiles = (M / E::TM) * (N / E::TN);
  hipLaunchKernelGGL(k_urgent_tiles<E>, dim3(tiles), dim3(E::THREADS), 0, st, A, B, C, M, N, K,
                     start_gt, end_gt);
  APK_LAUNCHED();
  return APK_OK;
}

template <class E>
static int occupancy_of(int* out) {
  APK_REQUIRE(out != nullptr, "occupancy: out is NULL");
  int n = 0;
  APK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_persistent_gemm<E>,
                                                       E::THREADS, 0));
  *out = n;
  return APK_OK;
}

}  // namespace apk

extern "C" int apk_persistent_gemm(int engine, const void* A, const void* B,
                                   float* C, int M, int N, int K, int k_chunk,
                                   unsigned int* next_task, apk_tile_record* log,
                                   int blocks, void* stream) {
  using namespace apk;
  switch (engine) {
    case APK_ENGINE_VALU64:
      return launch_persistent_gemm<EngValu64>(A, B, C, M, N, K, k_chunk,
                                               next_task, log, blocks,
                                               as_stream(stream));
    case APK_ENGINE_MFMA128:
      // Stage pairs (one barrier per 64 k) for tiles of whole pairs, except
      // where per-chunk records are asked for at chunks that end inside a pair.
      if (K % (2 * EngMfma128Pairs::KS) == 0 &&
          (log == nullptr || k_chunk % (2 * EngMfma128Pairs::KS) == 0))
        return launch_persistent_gemm<EngMfma128Pairs>(A, B, C, M, N, K, k_chunk,
                                                       next_task, log, blocks,
                                                       as_stream(stream));
      return launch_persistent_gemm<EngMfma128>(A, B, C, M, N, K, k_chunk,
                                                next_task, log, blocks,
                                                as_stream(stream));
    case APK_ENGINE_BF16X256:
      return launch_persistent_gemm<EngBf16x256>(A, B, C, M, N, K, k_chunk,
                                                 next_task, log, blocks,
                                                 as_stream(stream));
    case APK_ENGINE_BF16X128:
      return launch_persistent_gemm<EngBf16x128>(A, B, C, M, N, K, k_chunk,
                                                 next_task, log, blocks,
                                                 as_stream(stream));
    case APK_ENGINE_BF16X256X128:
      return launch_persistent_gemm<EngBf16x256x128>(A, B, C, M, N, K, k_chunk,
                                                    next_task, log, blocks,
                                                    as_stream(stream));
    default:
      set_error("persistent_gemm: unknown engine %d", engine);
      return APK_EINVAL;
  }
}

extern "C" int apk_persistent_gemm_occupancy(int engine, int* blocks_per_cu) {
  using namespace apk;
  switch (engine) {
    case APK_ENGINE_VALU64: return occupancy_of<EngValu64>(blocks_per_cu);
    case APK_ENGINE_MFMA128: {
      // the smaller of the two ring shapes' occupancies (both 1 per CU)
      int a = 0, b = 0;
      const int rc = occupancy_of<EngMfma128>(&a);
      if (rc != APK_OK) return rc;
      const int rc2 = occupancy_of<EngMfma128Pairs>(&b);
      if (rc2 != APK_OK) return rc2;
      *blocks_per_cu = a < b ? a : b;
      return APK_OK;
    }
    case APK_ENGINE_BF16X256: return occupancy_of<EngBf16x256>(blocks_per_cu);
    case APK_ENGINE_BF16X128: return occupancy_of<EngBf16x128>(blocks_per_cu);
    case APK_ENGINE_BF16X256X128: return occupancy_of<EngBf16x256x128>(blocks_per_cu);
    default:
      set_error("occupancy: unknown engine %d", engine);
      return APK_EINVAL;
  }
}

extern "C" int apk_persistent_gemm_noalloc(int engine, const void* A, const void* B, float* C,
                                           int M, int N, int K, int k_chunk,
                                           apk_tile_record* log, int blocks, void* stream) {
  using namespace apk;
  int rc;
  switch (engine) {
    case APK_ENGINE_VALU64:
      rc = validate_persistent_gemm<EngValu64>(A, B, C, M, N, K, k_chunk, blocks);
      break;
    case APK_ENGINE_MFMA128:
      rc = validate_persistent_gemm<EngMfma128>(A, B, C, M, N, K, k_chunk, blocks);
      break;
    case APK_ENGINE_BF16X256:
      rc = validate_persistent_gemm<EngBf16x256>(A, B, C, M, N, K, k_chunk, blocks);
      break;
    case APK_ENGINE_BF16X128:
      rc = validate_persistent_gemm<EngBf16x128>(A, B, C, M, N, K, k_chunk, blocks);
      break;
    case APK_ENGINE_BF16X256X128:
      rc = validate_persistent_gemm<EngBf16x256x128>(A, B, C, M, N, K, k_chunk, blocks);
      break;
    default:
      set_error("persistent_gemm_noalloc: unknown engine %d", engine);
      return APK_EINVAL;
  }
  if (rc != APK_OK) return rc;
  unsigned* q = nullptr;
  rc = scratch_of_current_device(&q);
  if (rc != APK_OK) return rc;
  hipLaunchKernelGGL(k_zero_words, dim3(1), dim3(64), 0, as_stream(stream), q,
                     (int)APK_QUEUE_WORDS);
  APK_LAUNCHED();
  return apk_persistent_gemm(engine, A, B, C, M, N, K, k_chunk, q, log, blocks, stream);
}

extern "C" int apk_urgent_gemm(int engine, const void* A, const void* B, float* C, int M, int N,
                               int K, long long* start_gt, unsigned long long* end_gt,
                               void* stream) {
  using namespace apk;
  switch (engine) {
    case APK_ENGINE_VALU64:
      return launch_urgent_tiles<EngValu64>(A, B, C, M, N, K, start_gt, end_gt, as_stream(stream));
    case APK_ENGINE_MFMA128:
      if (K % (2 * EngMfma128Pairs::KS) == 0)
        return launch_urgent_tiles<EngMfma128Pairs>(A, B, C, M, N, K, start_gt, end_gt,
                                                    as_stream(stream));
      return launch_urgent_tiles<EngMfma128>(A, B, C, M, N, K, start_gt, end_gt, as_stream(stream));
    case APK_ENGINE_BF16X256:
      return launch_urgent_tiles<EngBf16x256>(A, B, C, M, N, K, start_gt, end_gt, as_stream(stream));
    case APK_ENGINE_BF16X128:
      return launch_urgent_tiles<EngBf16x128>(A, B, C, M, N, K, start_gt, end_gt, as_stream(stream));
    case APK_ENGINE_BF16X256X128:
      return launch_urgent_tiles<EngBf16x256x128>(A, B, C, M, N, K, start_gt, end_gt,
                                                 as_stream(stream));
    default:
      set_error("urgent_gemm: unknown engine %d", engine);
      return APK_EINVAL;
  }
}
