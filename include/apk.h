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
 *  VALU64   : 64x64 fp32 tile, 256 threads, one fmaf chain per output in the
 *             reference's k order (src/tile.cuh:62-107) -- bit-identical to a
 *             correctly rounded sequential fmaf over k.
 *  MFMA128  : 128x128 fp32 tile on v_mfma_f32_32x32x2_f32 (fp32 matrix
 *             cores), 256 threads, 3-stage LDS ring fed by buffer_load ... lds.
 *  BF16X256 : 256x256 tile of a bf16 GEMM with fp32 accumulation on
 *             v_mfma_f32_32x32x16_bf16, 512 threads (two waves per SIMD),
 *             1 block per CU (replaces the reference's fp16 wmma tile,
 *             src/tcyield.cu:91-356). Operands are bf16 (uint16 bit
 *             patterns): A is M x K row-major and B is passed TRANSPOSED, as
 *             Bt = N x K row-major (C = A . Bt^T); C is fp32 M x N. 32-deep
 *             k-stages in pairs (sites every 64 k): K must be a multiple
 *             of 64.
 *  BF16X128 : 128x128 tile of the same bf16 GEMM (same operand layout) on
 *             ONE wave (64 threads), 32 KiB of LDS: 4 blocks per CU, where
 *             the 256x256 tile cannot run (configs[4] of the reference's
 *             study at 4 blocks/CU). K must be a multiple of 32. At 4
 *             blocks per CU its preemptible kernels take every register
 *             of every SIMD: generations must be raised by the grid's own
 *             setter (flag_set/sched), since apk_raise_flag's kernel finds
 *             no SIMD until blocks exit.
 *  BF16X256X128 : 256x128 tile (256 rows of A, 128 of Bt) of the same bf16
 *             GEMM on 256 threads, 48 KiB of LDS: 2 blocks per CU
 *             (configs[4] at 2 blocks/CU). K must be a multiple of 32.
 * Both take 16-deep k-stages in pairs (sites every 32 k). Every bf16 engine
 * forms each output's sum in the same k order: their C is bit-identical to
 * each other's on the same operands.
 * For the fp32 engines A is M x K and B is K x N, row-major fp32.
 */
enum {
  APK_ENGINE_VALU64 = 0,
  APK_ENGINE_MFMA128 = 1,
  APK_ENGINE_BF16X256 = 2,
  APK_ENGINE_BF16X128 = 3,
  APK_ENGINE_BF16X256X128 = 4,
  APK_ENGINE_COUNT = 5
};

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
  int elem_bytes;         /* operand element size: 4 = fp32, 2 = bf16 */
  int b_transposed;       /* 1: B is passed as Bt (N x K row-major) */
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
 * workers pops output tiles from the work queue next_task (APK_QUEUE_WORDS
 * counters, 0 at launch) until all tilesM*tilesN tiles are taken. Each tile computes
 * C[tile] = A[rows, 0:K] . B[0:K, cols] with A MxK, B KxN, C MxN row-major
 * fp32 (lda = K, ldb = N, ldc = N). The reference's task is one tile with
 * per-task K; here K may be split into K/k_chunk chunks walked in order by
 * the same worker, and `log` (optional, may be NULL) receives one record per
 * (tile, chunk): log[tile * (K/k_chunk) + chunk]. k_chunk == K reproduces the
 * reference exactly. Requires M % tile_m == 0, N % tile_n == 0,
 * K % k_chunk == 0, k_chunk % k_stage == 0. */
int apk_persistent_gemm(int engine, const void* A, const void* B, float* C,
                        int M, int N, int K, int k_chunk,
                        unsigned int* next_task, apk_tile_record* log,
                        int blocks, void* stream);

/* urgent_tile (src/urgent_baseline.cu:100-112): the urgent job as one block
 * per output tile, block b computing tile b (row-major tile order) over the
 * whole K, with no work queue (nothing to clear, nothing allocated). Same
 * operands, layouts and per-element k order as apk_persistent_gemm, so C is
 * bit-identical to it. Optional outputs (device memory, may be NULL):
 * *start_gt = wall-clock ticks at block 0's first instruction (the
 * reference's uStartGT); *end_gt raised (atomic max, unsigned) to the time
 * each block's tile is stored (the reference's uEndGT; the caller zeroes
 * it). Requires M % tile_m == 0, N % tile_n == 0, K % k_stage == 0. */
int apk_urgent_gemm(int engine, const void* A, const void* B, float* C, int M, int N, int K,
                    long long* start_gt, unsigned long long* end_gt, void* stream);

/* Allocation-free variant of apk_persistent_gemm. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops). Same arguments and results as
 * apk_persistent_gemm minus next_task: the work-queue counters (APK_QUEUE_WORDS
 * unsigned) live in a file-scope device array of APK_NOALLOC_SCRATCH_WORDS
 * words (256 bytes) that every GPU the library runs on holds until the process
 * ends. Its size does not depend on the GEMM, so no input can exceed it; the
 * arguments are checked as for apk_persistent_gemm (same errors). Each call
 * first clears the counters with a one-wave kernel on `stream`, then launches
 * the GEMM on it; the function calls no hipMalloc, hipFree or other allocating
 * routine (the first call on a device looks up the array's device address
 * with hipGetSymbolAddress). All calls on one GPU share the array: calls that
 * overlap on one GPU (different streams, or different host threads) race and
 * must be serialised by the caller; calls in order on one stream are safe. */
#define APK_NOALLOC_SCRATCH_WORDS 64
int apk_persistent_gemm_noalloc(int engine, const void* A, const void* B, float* C,
                                int M, int N, int K, int k_chunk, apk_tile_record* log,
                                int blocks, void* stream);

/* ------------------------------------------------------------------------
 * Preemptible persistent GEMM (cooperative arm).
 *
 * Poll sites: APK_POLL_CHUNK polls at every poll_every-th k-chunk boundary of
 * a tile (the tile-boundary yield points of src/yield.cu:125-136 once K is
 * walked in chunks); APK_POLL_STAGE polls at every LDS k-stage (the
 * mid-pipeline points of src/midyield.cu:246-290). Sites sit at the stage
 * loop's barriers: the BF16X256 engine synchronises once per pair of
 * k-stages, so its site stride is rounded up to 2 stages (64 k). The flag is
 * sampled by a direct-to-LDS load issued right behind a stage's data loads
 * and retired by the same stage wait, so a poll never stalls the pipeline;
 * the value acted on is one k-stage (one pair) old.
 *
 * On a new generation every block logs its observation time; blocks that pop
 * an urgent tile from the event's mini-queue (src/yield.cu:155-183) yield:
 * they drain their in-flight stage loads, checkpoint per `resume`, run urgent
 * tiles through the same LDS ring until the mini-queue is empty, restore and
 * continue the interrupted tile. At a site before stage s, stages s and s+1
 * are resident in LDS and not yet computed (the "live" stages).
 *   APK_RESUME_CKPT_FULL : accumulators + the live LDS stages -> HBM -> back
 *   APK_RESUME_CKPT_ACC  : accumulators -> HBM -> back; live stages re-fetched
 *   APK_RESUME_RESTART   : abandon the tile, restart it from k = 0 (the
 *                          reference's semantics, src/midyield.cu:237-258)
 * All three produce bit-identical C: the per-tile k order never changes.
 *
 * APK_POLL_ISSUE is the window-forcing site of the drain experiment
 * (src/midyield.cu:246-258): the flag is sampled as for APK_POLL_STAGE, but a
 * new generation is acted on at the top of the NEXT stage iteration, right
 * after the compute that issued the following stage's loads and before any
 * wait, so both live stages may still be in flight. Every block that sees
 * the generation checkpoints at once (drain: after vmcnt(0); naive: without
 * it) and only then pops the event's mini-queue; blocks that get no urgent
 * tile continue with their state intact. Cooperative arm only, device flag
 * only.
 */
enum { APK_POLL_OFF = 0, APK_POLL_CHUNK = 1, APK_POLL_STAGE = 2, APK_POLL_ISSUE = 3 };
/* The flag may be replicated so that no single address is polled by every
 * CU: copy c lives at byte offset c * APK_FLAG_STRIDE. */
#define APK_FLAG_STRIDE 4096
#define APK_FLAG_MAX_COPIES 256
/* Per-block statistics of the yield kernel, APK_STATS_PER_BLOCK u64 each. */
#define APK_STATS_PER_BLOCK 16
enum {
  APK_ST_YIELDS = 0,    /* cooperative yields served */
  APK_ST_SAVE = 1,      /* ticks spent checkpointing */
  APK_ST_URGENT = 2,    /* ticks spent on urgent tiles */
  APK_ST_RESTORE = 3,   /* ticks spent restoring */
  APK_ST_INFLIGHT = 4,  /* resumed checkpoints (served yields; at issue sites
                           every observer) at which a live stage was observed
                           still in flight when the drain (naive: the save)
                           began: the last direct-to-LDS load of the newest
                           stage had not yet written its LDS bytes */
  APK_ST_RETREATS = 5,  /* retreats (retreat arm) */
  APK_ST_RESUMED = 6,   /* resume-queue entries taken */
  APK_ST_ERRORS = 7,    /* resume-ring waits that ran out (a block holding an
                           entry stopped): entries never published in time
                           (lost), or entries never freed for a reserved
                           ticket; 0 in every correct run */
  APK_ST_STALE = 8,     /* resumed checkpoints holding LDS stages that differ
                           from the stages once every load had landed (naive
                           only); each resumes a wrong tile */
  APK_ST_CHECKPOINTS = 9, /* checkpoints taken (issue sites: every observer) */
  APK_ST_INFLIGHT_ALL = 10, /* APK_ST_INFLIGHT over every checkpoint taken */
  APK_ST_STALE_ALL = 11,    /* APK_ST_STALE over every checkpoint taken */
  APK_ST_DECLINED = 12,     /* retreats declined because the resume ring held
                               rq_capacity unreleased tickets (the block kept
                               its tile and worked on; nothing is lost) */
  APK_ST_START_SITES = 13   /* new flag values first seen at a task-start site
                               (cooperative arm, stage polls: the sample taken
                               with the task pop, before the tile's first
                               loads have landed) */
};

/* Work queue: every persistent kernel pops tasks from APK_QUEUE_WORDS
 * unsigned counters (zero at launch). The tiles are split into
 * APK_QUEUE_XCDS lists, one per XCD, each a compact 2-D region of the tile
 * grid; a worker pops from its own XCD's list first (so concurrently running
 * tiles share A and B panels in that XCD's L2) and steals from the others
 * when it is empty. Task u always computes tile u mod (tilesM * tilesN). */
#define APK_QUEUE_WORDS 16
#define APK_QUEUE_XCDS 8
/* Control words of the retreat arm's resume ring (apk_yield_params.rq_ctl). */
#define APK_RQ_CTL_WORDS 4
/* Dispatch domains of the retreat arm: a workgroup is dealt round-robin to
 * one of the 8 XCDs and then to one of its 4 shader engines, and runs only
 * on a CU of that shader engine. */
#define APK_SES_PER_XCD 4
#define APK_RETREAT_DOMAINS 32
enum { APK_RESUME_CKPT_FULL = 0, APK_RESUME_CKPT_ACC = 1, APK_RESUME_RESTART = 2 };

typedef struct apk_yield_params {
  /* background GEMM; tasks cycle the tile grid (src/urgent_baseline.cu:78-80) */
  const void* A;               /* element type and B layout per engine (above) */
  const void* B;
  float* C;
  int M, N, K, k_chunk;
  unsigned int num_tasks;      /* < 2^31 */
  unsigned int* next_task;     /* APK_QUEUE_WORDS counters, 0 at launch */
  /* urgent job: Cu (Mu x Nu) = Au (Mu x Ku) . Bu (Ku x Nu), split into tiles
   * that yielding blocks pop per event */
  const void* Au;
  const void* Bu;
  float* Cu;
  int Mu, Nu, Ku;
  int* uq_next;                /* [events] mini-queue counters, 0 at launch */
  /* generation flag and event bookkeeping (src/yield.cu:96-102); times are
   * device wall-clock ticks */
  const int* flag;             /* polled flag: 0 none, e events fired, -1 stop;
                                  flag_copies ints APK_FLAG_STRIDE bytes apart */
  int flag_copies;             /* copies of the flag (1..APK_FLAG_MAX_COPIES);
                                  block b polls copy b % flag_copies */
  int flag_system;             /* 1: flag is host-mapped memory (system scope) */
  int* flag_set;               /* device setter target (block 0) with the same
                                  copies; NULL = none */
  const long long* sched;      /* [events] cumulative ticks after the setter's first poll */
  int num_events;
  long long stop_after;        /* setter stores -1 this many ticks after the
                                  last scheduled event (0 = never) */
  int poll_every;              /* chunks between polls (APK_POLL_CHUNK) */
  long long* set_gt;           /* [events] */
  long long* obs_gt;           /* [events * blocks] */
  int* claim;                  /* [events] first popper + 1 */
  int* claim_site;             /* [events] k-stage of the claimer's yield */
  long long* u_gt;             /* [2 * events] urgent start / claimer end */
  unsigned long long* u_end_max; /* [events] last urgent tile completion */
  /* checkpoint */
  int resume;                  /* APK_RESUME_* */
  float* ckpt;                 /* blocks * apk_yield_ckpt_floats(engine) */
  int poison;                  /* detector control: +1.0 on one staged B value
                                  of every urgent tile (src/midyield.cu:146-147) */
  /* verification and statistics (each may be NULL) */
  unsigned long long* task_hash; /* [num_tasks] fingerprint of each completed task */
  unsigned long long* u_hash;    /* [events * urgent tiles] */
  unsigned long long* stats;     /* [blocks * APK_STATS_PER_BLOCK], APK_ST_*;
                                    added to (atomically) at block exit, so
                                    launches may share rows; 0 at launch */
  /* exactly-once oracle (used by the oracle instantiation only) */
  int* exec_count;             /* [num_tasks] */
  int* u_exec_count;           /* [events] */
  /* per-event urgent outputs: event e writes its tiles at Cu + e *
   * cu_event_stride floats (0 = every event overwrites Cu); the reference's
   * CuAll (src/midyield.cu:410-416) */
  long long cu_event_stride;
  /* 1 = skip the drain (vmcnt 0) before the checkpoint -- the reference's
   * "naive" discipline (src/midyield.cu:180-200) as a control experiment:
   * a live stage still in flight is checkpointed stale (APK_ST_STALE counts
   * it; the resumed tile then differs). 0 = drain. */
  int naive;
  /* run timeline (src/urgent_baseline.cu:66-88), may be NULL: run_gt[0] =
   * block 0's start, run_gt[1] = exit of the last block (0 at launch: the
   * latest exit is kept with an atomic max); exit_count counts the exits and must be
   * 0 at launch */
  long long* run_gt;
  unsigned int* exit_count;
  /* ---- retreat arm: hand CUs to a kernel queued on another stream ----
   * retreat = R > 0: the urgent kernel has R workgroups. The hardware deals
   * a kernel's workgroups round-robin to the XCDs and their shader engines
   * (APK_RETREAT_DOMAINS in all), starting wherever its pointers stand, and a
   * workgroup only runs on a CU of its own shader engine. So at generation
   * 1 ceil(R / 32) blocks of EVERY shader engine -- the first grid's first
   * ceil(R / 32) of each to start, as they register in the last row of
   * retreat_count -- and at each later generation the newest continuation
   * (launch_epoch), all of it, retreat (counted in retreat_count[(e-1) * 32 +
   * xcd * 4 + se]; 32 * ceil(R/32) blocks in all): they drain their loads,
   * checkpoint their tile into the resume queue (per `resume`: accumulators
   * + live LDS stages, accumulators only, or nothing = restart from k = 0)
   * and exit, so that the kernel waiting on another stream is dispatched
   * onto their CUs. Every
   * worker pops the resume queue before taking a new task, so the tile is
   * finished by whichever worker (of this launch or of a later relaunch on
   * any stream) pops its entry; its k order never changes. Only blocks that
   * may still retreat poll at every site; the others poll at the first stage
   * of each new task (so obs_gt, when given, logs them late). The urgent job
   * is not run inside this kernel (Au may be NULL). 0 = cooperative arm. */
  int retreat;
  int* retreat_count;            /* [(events + 1) * APK_RETREAT_DOMAINS], 0 at job start:
                                    rows 0..events-1 the retreats of each generation,
                                    row `events` the first grid's registrations */
  long long* retreat_gt;         /* [2 * events] or NULL: [2e] earliest checkpoint
                                    start (host sets INT64_MAX), [2e+1] latest exit (0) */
  unsigned int* rq_ctl;          /* resume queue tickets, 4 words: [0] head, [1] tail,
                                    [2] reserved tickets not yet claimed, [3] tickets
                                    reserved and not yet released; 0 at job start */
  int* rq_entry;                 /* [rq_capacity * 4], a ring: ticket t uses entry t %
                                    rq_capacity = {task, stage, seq, kind << 8 | domain
                                    (xcd * 4 + shader engine of the retreating block)};
                                    seq = t: free, t + 1: published, set to t + capacity
                                    once read back. At job start entry i holds seq = i. */
  float* rq_slots;               /* rq_capacity * apk_yield_ckpt_floats(engine) floats */
  unsigned int rq_capacity;      /* entries in the ring, at least 2 (APK_EINVAL
                                    otherwise). A retreat that finds rq_capacity
                                    tickets unreleased is declined before it takes a
                                    ticket (APK_ST_DECLINED; the block keeps its tile).
                                    Sizing: 32 * ceil(retreat / 32) entries hold one
                                    generation's retreats, so none is declined while
                                    each generation is resumed before the next. */
  int continuation;              /* 1: a relaunch joining a running job -- generations
                                    already raised when it starts are not acted on */
  int block_base;                /* this launch's first row in obs_gt columns and stats */
  int obs_stride;                /* obs_gt row length (0 = gridDim); obs_gt may be NULL */
  /* Retreat arm, which blocks hand over their CU at generation g: a launch
   * with continuation = 0 (the job's first grid) by the per-domain quota at
   * g = 1 only; a continuation with launch_epoch > 0 all of its blocks at the
   * first generation after launch_epoch (its blocks sit on the CUs the
   * previous generation freed, one per dispatch domain; it must complete for
   * the next continuation, queued behind it on one stream, to start); a
   * continuation with launch_epoch = 0 never. Set it to the generation a
   * continuation follows (the flag value when it is queued): the
   * continuation treats generations up to it as seen, even if a later one was
   * raised before it got its CUs. */
  int launch_epoch;
} apk_yield_params;

/* persistent_yield / persistent_midyield (src/yield.cu:95-204,
 * src/midyield.cu:92-320) on a gfx950 tile engine. `oracle` selects the
 * instantiation that counts executions. */
int apk_persistent_yield(int engine, int poll, int oracle,
                         const apk_yield_params* params, int blocks, void* stream);

/* Floats of checkpoint storage one block needs (accumulators + two LDS
 * stages). */
long long apk_yield_ckpt_floats(int engine);

/* Raise the generation flag from a stream: one wave stores `value` into
 * every copy of the flag (agent scope, flag_copies ints APK_FLAG_STRIDE
 * apart) and, if set_gt is not NULL, its device wall-clock tick into
 * *set_gt. Queued ahead of an urgent kernel on the urgent stream it is the
 * "urgent task submitted" signal of the retreat arm: it needs no LDS and few
 * registers, so it is dispatched beside a fully resident persistent grid.
 * Replaces the reference's host flag write (cudaMemcpyAsync of the flag on a
 * control stream, src/yield.cu:845-858). */
int apk_raise_flag(int* flag, int flag_copies, int value, long long* set_gt, void* stream);

/* Host<->device clock calibration probe (spin_flag, src/yield.cu:206-214):
 * one wave spins on *flag until it reads non-zero and stores the device
 * wall-clock tick of that read into out[0] and the value read into out[1].
 * system_scope = 1 for a host-mapped flag (the host-set mode), 0 for device
 * memory. The spin is bounded: after max_ticks (> 0) without a non-zero read
 * it stores out[0] = -1 and returns, so a flag the host never writes cannot
 * hang the GPU. out: 2 device (or host-mapped) long longs. */
int apk_spin_flag(const int* flag, int system_scope, long long max_ticks, long long* out,
                  void* stream);

/* Engine clock under load (the read-back of scripts/lock_clocks.sh:15-25,
 * taken on the device): `blocks` one-wave blocks, dealt round-robin to the
 * XCDs, each count shader-clock cycles (s_memtime) and wall-clock ticks
 * (s_memrealtime) over a window of window_ticks wall ticks, sleeping between
 * reads. out[4 b .. 4 b + 3] = cycles, ticks, XCD, start tick; the mean clock
 * of block b's CU is cycles / ticks x the wall-clock rate. Queue it on a
 * second stream while the kernel to be measured runs: it needs no LDS and one
 * wave, so it is dispatched beside a fully resident grid. */
int apk_clock_probe(long long* out, int blocks, long long window_ticks, void* stream);

/* Resident blocks per CU of the preemptible kernel. */
int apk_persistent_yield_occupancy(int engine, int poll, int* blocks_per_cu);

/* ------------------------------------------------------------------------
 * Scheduler oracle on tiny tasks (the cfg5 exactly-once oracle; the
 * reference's oracle instantiations count full tiles, src/yield.cu:570-667,
 * src/tcyield.cu:815-839). Every wave is a worker: it pops `batch` task ids
 * at a time from APK_QUEUE_WORDS fetch-add counters (one list per XCD,
 * stealing when its own is empty) and runs each task as one
 * v_mfma_f32_16x16x16_bf16: task t multiplies A tile t % pa by B tile
 * (t / pa) % pb (16x16 bf16 each; B tiles passed transposed, N x K). Between
 * the MFMA and the task's completion the wave checks the generation flag; a
 * wave that pops an urgent task of a new event saves its accumulator tile to
 * HBM, runs urgent tasks until the event's mini-queue is empty, restores and
 * completes. Wave 0 of block 0 raises the events on a device-clock schedule.
 * Completion: exec_count[t] += 1 and the task's fingerprint
 * mix64(v + t * 0x9E3779B97F4A7C15) -- v = the wrapping sum over lanes l and
 * registers j of mix64(bits(C[l][j]) + ((4l + j) << 32)) -- is added to
 * checksum[0]; urgent task id = e * urgent_per_event + u uses A tile
 * (7 id + 3) % pa and B tile (13 id + 5) % pb, adds
 * mix64(v + id * 0x9E3779B97F4A7C15 + 0xD1B54A32D192ED03) to checksum[1] and
 * u_exec_count[e] += 1. Before a wave exits it checks the flag once more, so
 * every raised event is served. */
typedef struct apk_tiny_params {
  unsigned int num_tasks;
  unsigned int* next_task;       /* APK_QUEUE_WORDS counters, 0 at launch */
  int batch;                     /* task ids per pop, >= 1 */
  const uint16_t* A;             /* pa tiles of 16x16 bf16, row-major (M x K) */
  const uint16_t* Bt;            /* pb tiles of 16x16 bf16, transposed (N x K) */
  int pa, pb;
  int* exec_count;               /* [num_tasks], 0 at launch */
  unsigned long long* checksum;  /* [2]: background, urgent; 0 at launch */
  int* flag;                     /* generation flag, 0 at launch */
  const long long* sched;        /* [num_events] cumulative ticks after the setter's start */
  int num_events;
  long long* set_gt;             /* [num_events] */
  int* uq_next;                  /* [num_events] urgent mini-queue counters, 0 */
  int urgent_per_event;
  int* u_exec_count;             /* [num_events], 0 */
  float* ckpt;                   /* [waves * 256]: one accumulator tile per wave */
  unsigned long long* stats;     /* [2]: yields, urgent tasks run; 0 at launch */
  float* c_debug;                /* NULL, or [n_debug * 256]: C of tasks t < n_debug, lane-major */
  unsigned int n_debug;
} apk_tiny_params;

/* Launch the tiny-task oracle on `blocks` blocks of 256 threads (4 waves);
 * blocks * 4 waves need blocks * 4 * 256 floats of ckpt. */
int apk_tiny_oracle(const apk_tiny_params* params, int blocks, void* stream);

/* ------------------------------------------------------------------------
 * Notification microbenchmark (visibility_poll, src/yield.cu:216-293): every
 * block loops {work_iters dependent FMAs; optionally one 16-byte read of a
 * DRAM-resident traffic buffer; barrier; thread 0 loads its flag copy with a
 * synchronous agent-scope load; block 0 sets events on schedule and stores -1
 * stop_after ticks after the last one; barrier; log a new generation}. The
 * flag-load round trip of thread 0 is also timed (load_ticks). Dynamic LDS
 * of lds_bytes pins residency to that of a tile kernel. */
typedef struct apk_vis_params {
  int* flag;                   /* flag_copies ints APK_FLAG_STRIDE apart */
  int flag_copies;
  const long long* sched;      /* [events] cumulative ticks */
  int num_events;
  long long stop_after;        /* ticks after the last event; must be > 0 */
  long long max_ticks;         /* hard per-block deadline after its start; must be > 0 */
  long long* set_gt;           /* [events] */
  long long* obs_gt;           /* [events * blocks] */
  int work_iters;
  int loaded;                  /* 1: read traffic each iteration */
  const float* traffic;        /* traffic_len float4 */
  int traffic_len;
  float* sink;                 /* [blocks * 256] */
  long long* iter_count;       /* [blocks] iterations run */
  long long* load_ticks;       /* [blocks * 2]: sum and max of flag-load ticks */
  int* block_domain;           /* optional [blocks]: xcd * APK_SES_PER_XCD + shader engine */
} apk_vis_params;

int apk_visibility(const apk_vis_params* params, int blocks, int lds_bytes, void* stream);

/* Resident blocks per CU of the visibility kernel with lds_bytes of LDS. */
int apk_visibility_occupancy(int lds_bytes, int* blocks_per_cu);

#ifdef __cplusplus
}
#endif

#endif /* APK_H_ */
