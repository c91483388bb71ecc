/* apk.h -- C ABI of the MI355X (gfx950) preemptible persistent-GEMM library.
 *
 * The reference (AyaanFaisal21/APK) has no library interface: every kernel
 * is launched from the main() of a single-file CUDA binary. Each entry point
 * below is the launch of one of those kernels, with the reference's kernel
 * arguments as plain device pointers and sizes (cited per function, paths
 * relative to the reference repository root). All pointers are device
 * pointers unless stated; `stream` is a hipStream_t passed as void* (NULL =
 * the null stream). Launches are asynchronous; every function returns
 * APK_OK or an error code and never exits the process (the reference's
 * CUDA_CHECK-and-exit lives in the host binaries, src/persistent.cu:41-49).
 */
#ifndef APK_H_
#define APK_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  APK_OK = 0,
  APK_EINVAL = 1,  /* bad argument: shape, alignment, engine, grid */
  APK_EHIP = 2,    /* HIP runtime error; apk_last_error() has the text */
  APK_ERANGE = 3   /* size beyond a documented maximum */
};

/* Tile engines (compute of one output tile).
 *  VALU64  : 64x64 fp32 tile, 256 threads, one fmaf chain per output in the
 *            reference's k order (src/tile.cuh:62-107) -- bit-identical to a
 *            correctly rounded sequential fmaf over k.
 *  MFMA128 : 128x128 fp32 tile on v_mfma_f32_32x32x2_f32 (fp32 matrix cores),
 *            256 threads, 3-stage LDS ring fed by buffer_load ... lds.
 */
enum { APK_ENGINE_VALU64 = 0, APK_ENGINE_MFMA128 = 1, APK_ENGINE_COUNT = 2 };

/* Per-step timing record; layout of TileRecord (src/tile.cuh:37-42). start
 * and end are device wall-clock ticks (s_memrealtime, rate in
 * apk_device_info.wall_clock_khz); smid is the hw slot (XCC/SE/CU bits). */
typedef struct apk_tile_record {
  int64_t start;
  int64_t end;
  int32_t smid;
  int32_t block;
} apk_tile_record;

typedef struct apk_device_info {
  char name[128];
  char arch[64];
  int cu_count;           /* multiProcessorCount */
  int wall_clock_khz;     /* hipDeviceAttributeWallClockRate */
  int clock_khz;          /* peak engine clock */
  int lds_per_cu;         /* bytes */
  int regs_per_cu;        /* 32-bit registers per CU */
  int xcc_count;          /* XCDs visible (cu_count / CUs per XCD) */
} apk_device_info;

typedef struct apk_engine_geometry {
  int tile_m, tile_n;     /* output tile */
  int k_stage;            /* k depth of one LDS stage */
  int threads;            /* block size */
  int lds_bytes;          /* static LDS per block */
} apk_engine_geometry;

/* Text of the last error raised in this thread. */
const char* apk_last_error(void);

/* Device properties used by the host harness (replaces the
 * cudaGetDeviceProperties reads at src/persistent.cu:112-115). */
int apk_get_device_info(int device, apk_device_info* out);

/* Geometry of a tile engine. */
int apk_engine_geometry_of(int engine, apk_engine_geometry* out);

/* Resident blocks per CU of the persistent_gemm kernel of `engine`
 * (replaces cudaOccupancyMaxActiveBlocksPerMultiprocessor,
 * src/urgent_baseline.cu:165-167). */
int apk_persistent_gemm_occupancy(int engine, int* blocks_per_cu);

/* persistent_gemm (src/persistent.cu:51-79): a persistent grid of `blocks`
 * workers pops output tiles from the fetch-add counter *next_task (must be 0
 * at launch) until tilesM*tilesN tiles are taken. Each tile computes
 * C[tile] = A[rows, 0:K] . B[0:K, cols] with A MxK, B KxN, C MxN row-major
 * fp32 (lda = K, ldb = N, ldc = N). The reference's task is one tile with
 * per-task K; here K may be split into K/k_chunk chunks walked in order by
 * the same worker, and `log` (optional, may be NULL) receives one record per
 * (tile, chunk): log[tile * (K/k_chunk) + chunk]. k_chunk == K reproduces the
 * reference exactly. Requires M % tile_m == 0, N % tile_n == 0,
 * K % k_chunk == 0, k_chunk % k_stage == 0. */
int apk_persistent_gemm(int engine, const float* A, const float* B, float* C,
                        int M, int N, int K, int k_chunk,
                        unsigned int* next_task, apk_tile_record* log,
                        int blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* APK_H_ */
