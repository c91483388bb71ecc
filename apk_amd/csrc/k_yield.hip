// k_yield.hip -- the preemptible persistent GEMM (cooperative arm).
//
// Counterpart of persistent_yield (reference src/yield.cu:95-204) and
// persistent_midyield (src/midyield.cu:92-320), rebuilt around the gfx950
// direct-to-LDS pipeline:
//  * workers pop output tiles from an HBM fetch-add queue (tasks cycle the
//    tile grid) and walk each tile's K in LDS k-stages;
//  * the generation flag is sampled by a direct-to-LDS load issued right
//    behind the data loads of a poll site's stage; the site's ordinary
//    "stage landed" wait retires it, so reading it costs one LDS read and
//    never a stall (the sample is one stage old);
//  * at poll sites (every poll_every chunks, or every stage) a new generation
//    is logged by every block; blocks that pop an urgent tile from the
//    event's mini-queue yield: drain, checkpoint (accumulators and the two
//    resident LDS stages to HBM), run urgent tiles through the same ring, restore,
//    continue -- the tile's k order is untouched, so C is bit-identical to an
//    unpreempted run;
//  * block 0 optionally acts as the device setter of a pre-scheduled event
//    train (src/yield.cu:186-195);
//  * retreat arm: instead of running the urgent job itself, a block that
//    wins one of the event's `retreat` slots checkpoints its tile into an
//    HBM resume queue and exits, handing its CU to a kernel queued on
//    another stream; every worker pops that queue before new tasks.
// Every branch that contains a barrier is taken on values all threads read
// from LDS after a barrier (the snapshot discipline of src/midyield.cu:
// 177-200), so a block never splits across barriers.
#include "capi.hpp"
#include "engine_bf16.hpp"
#include "engine_mfma128.hpp"
#include "engine_valu64.hpp"
#include "pipeline.hpp"

namespace apk {

// RETREAT selects the retreat arm (P.retreat > 0) at compile time, so the
// cooperative instantiations carry none of its code and the retreat ones
// none of the in-kernel urgent path.
template <class E, int POLL, bool ORACLE, bool SYS, bool RETREAT>
__global__ void __launch_bounds__(E::THREADS) __attribute__((amdgpu_waves_per_eu(E::MIN_WAVES_PER_SIMD, E::WAVES_PER_SIMD)))
k_persistent_yield(const apk_yield_params) {
  // Every parameter is re-read from the kernel-argument segment where it is
  // used (P() is opaque to the optimiser), instead of being loaded once at
  // entry and held in scalar registers for the whole kernel: the stage loop
  // then keeps its own values in registers without spilling.
  auto P = [&]() -> const KArg<apk_yield_params>& { return *kernel_args<apk_yield_params>(); };
  __shared__ __attribute__((aligned(16))) char ring[E::LDS_BYTES];
  // flag sample issued with stage t: [t % NS]; [NS]: the one issued with a
  // task pop (task-start sites)
  __shared__ int flagring[E::NS + 1];
  __shared__ unsigned s_u32;
  __shared__ int s_i32[3];
  __shared__ uint64_t s_red[E::THREADS / 64];

  // Block-wide counters of thread 0 (yields, times, retreats, ...) and the
  // setter's state live in LDS: they are touched only off the stage loop.
  __shared__ unsigned long long s_stats[APK_STATS_PER_BLOCK];
  __shared__ long long s_setter[2];  // next event, time base
  __shared__ long long s_serve_t1;   // start of the current service's urgent work
  __shared__ int s_fsync;            // synchronous flag read (syncPoll)

  const int tid = threadIdx.x, bid = blockIdx.x;
  // Values the stage loop does not need are recomputed from the parameters
  // where they are used rather than held across it.
  auto tilesN = [&] { return P().N / E::TN; };
  auto uTilesN = [&] { return P().Nu > 0 ? P().Nu / E::TN : 1; };
  auto nU = [&] {
    return (!RETREAT && P().Au && P().Mu > 0 && P().Nu > 0) ? (P().Mu / E::TM) * uTilesN() : 0;
  };
  auto ckslot = [&]() -> float* {
    return P().ckpt ? P().ckpt + (size_t)bid * Ckpt<E>::SLOT_FLOATS : nullptr;
  };
  auto copies = [&] { return P().flag_copies > 0 ? P().flag_copies : 1; };
  auto row = [&] { return P().block_base + bid; };  // this block's stats / obs column
  // Poll sites sit at barriers: every GROUP-th k-stage at the finest.
  // Chunk polls (APK_POLL_CHUNK) are at every poll_every-th k-chunk boundary
  // the block passes, counted across its tasks (src/yield.cu:124-134 polls
  // at every PE-th tile boundary): chunksDone counts the chunks of the
  // background tasks this block has completed.
  const int chunkStages = P().k_chunk / E::KS;
  const int pollEvery = POLL == APK_POLL_CHUNK && P().poll_every > 0 ? P().poll_every : 1;
  const int pollStride = [&] {
    const int st = (POLL == APK_POLL_STAGE || POLL == APK_POLL_ISSUE) ? 1
                                                                      : chunkStages * pollEvery;
    return (st + E::GROUP - 1) / E::GROUP * E::GROUP;
  }();
  int chunksDone = 0;  // uniform
  const i32x4 flag_rsrc =
      make_rsrc((const char*)P().flag + (size_t)(bid % copies()) * APK_FLAG_STRIDE, 4);
  const bool isSetter = P().flag_set != nullptr && P().sched != nullptr && bid == 0;
  constexpr bool retreatArm = RETREAT && POLL != APK_POLL_OFF;
  // Task-start sites (cooperative arm, stage polls, drain discipline): thread
  // 0 samples the flag right before it takes a new task, so the sample lands
  // with the task pop's own round trip, and a new generation is acted on at
  // stage 0 before the tile's first loads have landed. Without it the first
  // site of a task reads a sample only once the first region is in, and that
  // wait is part of the stretch between two tasks in which a block sees
  // nothing -- the stretch the last observer of an event is found in.
  const bool startSites = POLL == APK_POLL_STAGE && !retreatArm && !P().naive;
  auto domain = [&] { return (int)xcc_id() * APK_SES_PER_XCD + (int)se_id(); };
  auto quota = [&] { return (P().retreat + APK_RETREAT_DOMAINS - 1) / APK_RETREAT_DOMAINS; };
  // Retreat arm: whether this block may still retreat at a later generation
  // (uniform). The first grid's blocks register in their (XCD, shader
  // engine) domain as they start, in the row of retreat_count after the
  // events' rows: the first ceil(R / 32) of each domain are the ones that
  // retreat at generation 1. A continuation that follows an earlier
  // generation retreats, all of it, at the next one. Blocks that may retreat
  // poll at every site; the others only at the first stage of each new task
  // (where the stop sentinel is seen), so the every-site polls cost the
  // background on 32 * ceil(R / 32) blocks instead of on all of them.
  bool mayRetreat = false;
  // The blocks that may retreat read the flag itself at their stage sites
  // (one load, one barrier) rather than the sample issued a stage (or a pair
  // of stages) earlier, to act that much sooner.
  bool syncPoll = false;
  const int* myFlag = (const int*)((const char*)P().flag + (size_t)(bid % copies()) * APK_FLAG_STRIDE);

  const uint32_t wl = wave_lds(ring);
  const uint32_t flag_lds = lds_addr_of(flagring);
  if (tid <= E::NS) flagring[tid] = 0;
  if (tid < APK_STATS_PER_BLOCK) s_stats[tid] = 0;
  if (tid < 2) s_setter[tid] = 0;
  if (P().run_gt && bid == 0 && tid == 0) P().run_gt[0] = wall_ticks();
  __syncthreads();
  if constexpr (retreatArm) {
    if (P().continuation == 0) {
      if (tid == 0)
        s_u32 = (unsigned)fetch_add_i32(
            &P().retreat_count[(size_t)P().num_events * APK_RETREAT_DOMAINS + domain()], 1);
      __syncthreads();
      mayRetreat = (int)uniform(s_u32) < quota();
      __syncthreads();
    } else {
      mayRetreat = P().launch_epoch > 0 && P().launch_epoch < P().num_events;
    }
  }

  int lastSeen = 0;     // uniform: every thread derives it from the same samples
  int fLatest = 0;      // freshest landed sample, for the task-boundary stop check
  if (POLL != APK_POLL_OFF && P().continuation) {
    // A relaunch joins a running job: generations raised before it started
    // were handled by the blocks that saw them.
    if (tid == 0)
      s_u32 = (unsigned)(SYS ? __hip_atomic_load(P().flag, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_SYSTEM)
                             : flag_load(P().flag));
    __syncthreads();
    const int f0 = (int)uniform(s_u32);
    __syncthreads();
    // A retreat-arm continuation starts from the generation it follows
    // (launch_epoch), so that one raised before it got its CUs still counts.
    if (f0 < 0) fLatest = f0;
    else lastSeen = proto::first_seen(f0, P().launch_epoch, P().num_events);
  }
  enum { ST_YIELDS = APK_ST_YIELDS, ST_SAVE = APK_ST_SAVE, ST_URGENT = APK_ST_URGENT,
         ST_RESTORE = APK_ST_RESTORE, ST_INFLIGHT = APK_ST_INFLIGHT,
         ST_RETREATS = APK_ST_RETREATS, ST_RESUMED = APK_ST_RESUMED, ST_ERRORS = APK_ST_ERRORS,
         ST_STALE = APK_ST_STALE, ST_CHECKPOINTS = APK_ST_CHECKPOINTS,
         ST_DECLINED = APK_ST_DECLINED, ST_START_SITES = APK_ST_START_SITES,
         ST_INFLIGHT_ALL = APK_ST_INFLIGHT_ALL, ST_STALE_ALL = APK_ST_STALE_ALL };
  auto stat = [&](int k, uint64_t v) { s_stats[k] += v; };  // thread 0 only

  auto set_flag = [&](int v) {
    for (int c = 0, n = copies(); c < n; ++c)
      flag_store((int*)((char*)P().flag_set + (size_t)c * APK_FLAG_STRIDE), v);
  };

  // Broadcast a value thread 0 computed (uniform afterwards).
  auto bcast = [&](unsigned v) -> unsigned {
    if (tid == 0) s_u32 = v;
    lds_sync();
    const unsigned r = uniform(s_u32);
    lds_sync();
    return r;
  };

  auto pop_urgent = [&](int ev) -> int {
    unsigned v = 0;
    if (tid == 0) v = (unsigned)fetch_add_i32(&P().uq_next[ev], 1);
    return (int)bcast(v);
  };

  // A job is one output tile through the stage loop below: a background
  // task (from the resume queue or the work queue), preemptible at poll
  // sites; or, while the block serves event `serving`, one tile of that
  // event's urgent GEMM (its own A, B, C and K; not preemptible). A service
  // ends with the interrupted background tile re-entering from its
  // checkpoint. Urgent tiles go through the same loop, so the kernel holds
  // one software pipeline and one epilogue, not two of each.
  enum { FRESH = 0, ACC = 1, FULL = 2, AS_IS = 3 };
  int serving = -1;        // event this block serves, or -1
  int uidx = 0;            // while serving: the urgent tile of the next job
  unsigned savedTask = 0;  // while serving: the interrupted background task,
  int savedStage = 0;      // its stage and how it re-enters
  int savedKind = FRESH;

  for (;;) {
    if (POLL != APK_POLL_OFF && serving < 0 && fLatest < 0) break;  // host stop sentinel
    // Reconverge before the thread-0 pop: without a barrier here the
    // compiler may thread the previous iteration's thread-0 regions into
    // this one across the back-edge and split the block's lanes over two
    // loop iterations (lanes 1..63 spinning on a stale task at the barrier
    // below while lane 0 waits outside the loop to pop the next one).
    lds_sync();

    // ---- the next job ----
    // The stage loop is (re)entered with the tile's state taken from:
    //   FRESH   start at k = 0 (new task, urgent tile, or a restart);
    //   ACC     accumulators from `src`; stages s, s+1 fetched again;
    //   FULL    accumulators and the two live stages from `src`;
    //   AS_IS   nothing to do: the loop left at a poll site with its state
    //           intact (the site found nothing to yield for).
    unsigned task = 0;
    int srcKind = FRESH, s = 0, siteDone = -1;
    const float* src = nullptr;
    bool urgent = false;
    int rqHeld = -1;  // resume ticket whose checkpoint this job reads back
    bool startSite = false;  // uniform: a task-start sample was taken for this job
    int fStart = 0;          // uniform: its value
    if (!RETREAT && serving >= 0) {
      if (uidx < nU()) {
        urgent = true;
      } else {
        // Every urgent tile of the event is taken: the service ends and the
        // interrupted tile re-enters at the site it left (not polled again).
        if (tid == 0) {
          const int64_t t2 = wall_ticks();
          atomic_max_u64(&P().u_end_max[serving], (unsigned long long)t2);
          P().u_gt[2 * (size_t)serving + 1] = t2;
          stat(ST_YIELDS, 1);
          stat(ST_URGENT, (uint64_t)(t2 - s_serve_t1));
        }
        task = savedTask;
        srcKind = savedKind;
        if (savedKind != FRESH) {
          s = savedStage;
          siteDone = savedStage;
          src = ckslot();
        }
        serving = -1;
      }
    } else {
      // Thread 0 takes the next task: a checkpointed tile from the resume
      // queue first (retreat arm), else a new task from the work queue.
      // kind: -1 new task; 0 restart from k = 0; 1 resume from the saved
      // accumulators at the saved stage; 2 the same plus the live stages.
      if (tid == 0) {
        unsigned t = 0xffffffffu;
        int kind = -1, st = 0, tk = 0;
        if constexpr (retreatArm) {
          const unsigned q = rq_pop(P().rq_ctl);
          if (q != RQ_NONE) {
            int* en = P().rq_entry + (size_t)(q % P().rq_capacity) * 4;
            const int ready = rq_wait_ready(en, q);
            if (ready > 0) {
              t = (unsigned)en[0];
              st = en[1];
              kind = ready - 1;
              tk = (int)q;
              stat(ST_RESUMED, 1);
              // a restart entry carries no checkpoint: free it at once
              if (kind == 0) rq_release(P().rq_ctl, en, q, P().rq_capacity);
            } else {
              stat(ST_ERRORS, 1);  // never published within the deadline: the task is lost
              t = 0xfffffffeu;
            }
          }
        }
        if (t == 0xffffffffu) {
          // the task-start sample goes out in front of the pop's fetch-add,
          // and the wait for the pop retires it
          if (startSites) sample_flag<SYS>(flag_rsrc, flag_lds + 4u * (uint32_t)E::NS);
          t = TaskQueue(P().next_task, P().M / E::TM, tilesN(), P().num_tasks).pop((int)xcc_id());
          if (startSites) wait_vmcnt<0>();
        }
        s_u32 = t;
        s_i32[0] = kind;
        s_i32[1] = st;
        s_i32[2] = tk;
      }
      __syncthreads();
      task = uniform(s_u32);
      const int kind = uniform(s_i32[0]);
      const int qStage = uniform(s_i32[1]);
      const int qTicket = uniform(s_i32[2]);
      if (startSites && kind < 0) {
        startSite = true;
        fStart = uniform(flagring[E::NS]);
      }
      __syncthreads();
      if (task == 0xfffffffeu) continue;  // lost resume entry (counted)
      if (task >= P().num_tasks) break;
      if (retreatArm && kind > 0) {
        src = P().rq_slots + (size_t)((unsigned)qTicket % P().rq_capacity) * Ckpt<E>::SLOT_FLOATS;
        s = qStage;
        srcKind = kind;
        rqHeld = qTicket;
      }
    }

    // The job's operands and output tile.
    const typename E::Ctx ctx = urgent ? E::make_ctx(P().Au, P().Bu, P().Mu, P().Nu, P().Ku)
                                       : E::make_ctx(P().A, P().B, P().M, P().N, P().K);
    const int S = (urgent ? P().Ku : P().K) / E::KS;
    int row0, col0;
    if (urgent) {
      row0 = (uidx / uTilesN()) * E::TM;
      col0 = (uidx % uTilesN()) * E::TN;
    } else {
      const int tile = (int)(task % (unsigned)((P().M / E::TM) * tilesN()));
      row0 = (tile / tilesN()) * E::TM;
      col0 = (tile % tilesN()) * E::TN;
    }
    const bool pollable = POLL != APK_POLL_OFF && !urgent;
    const typename E::Lane ln = E::lane_offsets(ctx, row0, col0);
    typename E::Acc acc;
    int slot = 0, nextSite = 0, lastSlot = -1;
    // Pipelined pairs: the last computed pair's deferred k-step (its
    // operands in `tail`) runs at the start of the next pair's call, or
    // before the epilogue; a call that stops at a site has run it.
    typename TailFrag<E>::type tail;
    bool hasTail = false;  // uniform
    // Not at issue sites, whose loop issues the next pair ahead of the poll.
    constexpr bool kPipe = PipelinedPairs<E>::value && POLL != APK_POLL_ISSUE;

    // Poll sites are the stages s with s % pollStride == 0; `nextSite` is the
    // next one not yet passed (an urgent tile never reaches one), so a stage
    // costs two scalar compares. The sample a site s reads lands in
    // flagring[site_flag(slot of s)]: with one barrier per stage it is
    // issued in front of the data loads of stage s+1, right behind stage s's
    // own loads, so the ordinary "stage s landed" wait retires it too; with
    // one barrier per pair it goes out in front of the pair's loads, which
    // are all waited for. For a site at the tile's last stage the sample
    // goes out in front of the refetch that stands in for stage S.
    auto site_flag = [](int sl) { return E::GROUP == 1 ? next_slot<E>(sl) : sl; };
    auto sample = [&](int idx) {
      if (POLL != APK_POLL_OFF) {
        sample_flag<SYS>(flag_rsrc, flag_lds + 4u * (uint32_t)idx);
        lastSlot = idx;
      }
    };
    auto issue_stage = [&](int t, int tslot) {
      issue_loads<E>(ctx, ln, E::stage_dst(wl, ctx, tslot, t, S));
    };

    bool retreated = false, yielded = false;
    // Issue sites (APK_POLL_ISSUE): right after the barrier of stage s the
    // loads of stage s+2 (pair s+2, s+3) go out at once, and the site is
    // polled right behind them -- the window-forcing geometry of
    // src/midyield.cu:246-258: a checkpoint here holds a stage whose loads
    // were issued nanoseconds earlier. `ahead`: that issue is already done
    // for the current s (re-entry after a site, or a restored ring).
    bool ahead = false;
    // Stages resident or in flight, not yet computed, at a site before stage
    // st: what a FULL checkpoint keeps. With pairs the zero stage after an
    // odd tile's last stage is kept too (the pair is computed as a whole).
    auto live_at = [&](int st) -> int {
      if constexpr (POLL == APK_POLL_ISSUE)
        return E::GROUP == 2 ? E::NS : (S - st < E::NS ? S - st : E::NS);
      else
        return (E::GROUP == 2 || S - st >= 2) ? 2 : S - st;
    };
    int siteStride = pollStride;  // uniform: the gap between this job's sites
    for (;;) {  // (re)entries of the stage loop of this job
      if (srcKind != AS_IS) {
        syncPoll = retreatArm && !SYS && POLL == APK_POLL_STAGE && mayRetreat;
        siteStride = retreatArm && !mayRetreat ? S + 2 : pollStride;
        if (!pollable) {
          nextSite = S + 2;
        } else if (retreatArm && !mayRetreat) {
          nextSite = s == 0 ? 0 : S + 2;  // a new task's first stage only
        } else if (POLL == APK_POLL_CHUNK && pollEvery > 1) {
          // the next chunk boundary c at or after s whose running count
          // chunksDone + c is a multiple of poll_every
          const int c0 = (s + chunkStages - 1) / chunkStages;
          const int ph = (chunksDone + c0) % pollEvery;
          const int st = (c0 + (ph ? pollEvery - ph : 0)) * chunkStages;
          nextSite = (st + E::GROUP - 1) / E::GROUP * E::GROUP;
        } else {
          nextSite = (s + pollStride - 1) / pollStride * pollStride;
        }
        const int64_t tIn = wall_ticks();
        ahead = POLL == APK_POLL_ISSUE && srcKind == FULL;
        if (srcKind == FRESH) {
          E::zero(acc);
          issue_stage(s, slot);
          if (pollable) sample(site_flag(slot));  // s is a site
          issue_stage(s + 1, next_slot<E>(slot));
          if (urgent && P().poison) {
            // Test hook: corrupt the staged B[0][col0] of the urgent tile.
            wait_landed<E>();
            lds_sync();
            if (tid == 0) *(float*)(ring + E::A_STAGE) += 1.0f;
            lds_sync();
          }
        } else {
          // Accumulators hold stages [0, s); stages s, s+1 (issue sites: every
          // live stage) go to ring slots slot, slot+1, ... (from the
          // checkpoint, or s, s+1 fetched again), and the site at s gets a
          // fresh sample. A resume-queue slot was written by another block,
          // maybe on another XCD: acquire at agent scope (an invalidate of
          // this XCD's L2) before reading it. The cooperative arm reads back
          // what the same threads stored to the same addresses, which needs
          // no fence, and an L2 invalidate per wave would also drop the
          // operand panels the XCD's other blocks are reading.
          if constexpr (retreatArm) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
          Ckpt<E>::load_acc(acc, src);
          if (srcKind == FULL) {
            Ckpt<E>::load_ring(ring, src, slot, live_at(s));
            // The sample alone: the live slots now hold restored stages.
            sample(site_flag(slot));
            // Issue sites: the restored ring includes the stage(s) the next
            // iteration would issue; send the sample that goes with them.
            if constexpr (POLL == APK_POLL_ISSUE)
              sample(E::GROUP == 1 ? slot_after_next(slot) : (slot ^ 2));
            wait_vmcnt<0>();
            __syncthreads();  // restored ring visible to all waves
          } else {
            issue_stage(s, slot);
            sample(site_flag(slot));
            issue_stage(s + 1, next_slot<E>(slot));
          }
          if (tid == 0 && src == ckslot()) stat(ST_RESTORE, (uint64_t)(wall_ticks() - tIn));
          if constexpr (retreatArm) {
            if (rqHeld >= 0) {
              // every thread's reads of the entry's checkpoint have completed
              // (load_acc / the ring restore wait for them): free the entry
              __syncthreads();
              if (tid == 0)
                rq_release(P().rq_ctl,
                           P().rq_entry + (size_t)((unsigned)rqHeld % P().rq_capacity) * 4,
                           (unsigned)rqHeld, P().rq_capacity);
              rqHeld = -1;
            }
          }
        }
      }

      // The stage loop itself only notices a new generation and leaves; the
      // event log, the setter, the yield decision and the checkpoint all
      // happen below, outside it, so that none of their state is live in it.
      bool atSite = false;
      bool startHit = false;  // uniform: this site is a task-start site
      int fSeen = 0;
      if (startSite) {
        // Task-start site: stage 0's site, taken on the sample that came back
        // with the task pop, before the first loads have landed (they are in
        // flight; a yield drains them). Nothing new: stage 0's own site still
        // reads its sample.
        startSite = false;
        fLatest = fStart;
        if (fStart != lastSeen) {
          fSeen = fStart;
          atSite = true;
          startHit = true;
        }
      }
      while (!atSite && s < S) {
        if constexpr (E::GROUP == 1) {
          wait_landed<E>();
          lds_sync();
        }
        // Poll site: the flag sample for site s has landed with stage s (it
        // was issued in front of the loads of stage s+1, or of the pair s).
        // A new generation (or the setter's turn) ends the loop here, before
        // stage s is computed. With one barrier per stage the flag is read
        // right after the barrier; with pairs it is read in the engine's
        // `pre` hook (measured: 10.8% -> 7-9% every-site overhead for the
        // bf16 engine, while the same placement cost the fp32 engines 1-2%).
        if constexpr (E::GROUP == 1) {
          if constexpr (POLL == APK_POLL_ISSUE) {
            // Stage s+2 (and the sample for the site at s+1) at once, into the
            // slot of stage s-1, which every wave finished before the barrier.
            if (!ahead) {
              const int a = slot_after_next(slot);
              if (pollable) sample(a);
              issue_loads<E>(ctx, ln, E::stage_dst(wl, ctx, a, s + 2, S));
            }
            ahead = false;
          }
          if (POLL != APK_POLL_OFF && s == nextSite) {
            if (s != siteDone) {
              int f = uniform(flagring[site_flag(slot)]);
              if (syncPoll) {
                // The blocks that retreat at the next generation read the
                // flag itself at the site (one load and one barrier) instead
                // of the sample issued a stage earlier.
                if (tid == 0) s_fsync = flag_load(myFlag);
                lds_sync();
                f = uniform(s_fsync);
              }
              fLatest = f;
              if (f != lastSeen || isSetter) {
                fSeen = f;
                atSite = true;
                ahead = POLL == APK_POLL_ISSUE;
                break;
              }
            }
            nextSite += siteStride;
          }
          const int aheadSlot = slot_after_next(slot);
          const bool carry = s + 1 == nextSite;  // s+1 is a site
          // Stage s+2 (and the sample for a site at s+1) goes out under stage
          // s's matrix work; its slot held stage s-1, which every wave
          // finished before the barrier above.
          const typename E::Dst d = E::stage_dst(wl, ctx, aheadSlot, s + 2, S);
          E::compute(ring, slot, acc, [] { return true; }, [&](int i) {
            if constexpr (POLL != APK_POLL_ISSUE) {
              if (i == 0 && carry) sample(aheadSlot);
              E::issue_one(ctx, ln, d, i);
            }
          });
          slot = next_slot<E>(slot);
          ++s;
        } else {
          // Everything scalar about this pair -- the site bookkeeping and the
          // next pair's load descriptors -- is formed before the wait, while
          // the pair's loads land, and the descriptors are pinned there:
          // formed after the barrier (where the compiler sinks them in the
          // polled kernels, next to their use) they held back the next
          // pair's loads and cost the chunk-poll kernel 5-6% with no site
          // polled at all.
          const bool site = POLL != APK_POLL_OFF && s == nextSite;
          const bool check = site && s != siteDone;
          if (site) nextSite += siteStride;
          auto poll = [&]() -> bool {
            if (!check) return true;
            int f = uniform(flagring[site_flag(slot)]);
            if (syncPoll) {  // as in the one-stage loop above
              if (tid == 0) s_fsync = flag_load(myFlag);
              lds_sync();
              f = uniform(s_fsync);
            }
            fLatest = f;
            if (f != lastSeen || isSetter) {
              fSeen = f;
              atSite = true;
              return false;
            }
            return true;
          };
          // Stages s and s+1 are computed as one group; stages s+2, s+3 (and
          // the sample for a site at s+2) go out under its first stage, into
          // the other half of the ring, which held the previous pair.
          const int other = slot ^ 2;
          const bool carry = s + 2 == nextSite;
          typename E::Dst d0 = E::stage_dst(wl, ctx, other, s + 2, S);
          typename E::Dst d1 = E::stage_dst(wl, ctx, other + 1, s + 3, S);
          E::pin(d0);
          if constexpr (!HasIssueGroup<E>::value) E::pin(d1);  // unused by region loads
          wait_landed<E>();
          lds_sync();
          if constexpr (POLL == APK_POLL_ISSUE) {
            // Issue sites: the next pair goes out at once, then the poll.
            if (!ahead) {
              if (carry) sample(other);
#pragma unroll
              for (int i = 0; i < E::GROUP * E::LOADS; ++i) issue_group_one<E>(ctx, ln, d0, d1, i);
            }
            ahead = false;
            if (!poll()) {
              ahead = true;
              break;
            }
            E::compute(ring, slot, acc);
          } else if constexpr (kPipe) {
            auto mid = [&](int i) {
              if (i == 0 && carry) sample(other);
              issue_group_one<E>(ctx, ln, d0, d1, i);
            };
            const bool had = hasTail;
            hasTail = false;  // a tail is run by the call, ahead of its site check
            // A block that may retreat here issues the next pair's first loads
            // after its check: leaving, it then has nothing in flight to drain.
            if (!E::compute_pl(ring, slot, acc, tail, had, !(syncPoll && check), poll, mid))
              break;
            hasTail = true;
          } else {
            if (!E::compute(ring, slot, acc, poll, [&](int i) {
                  if (i == 0 && carry) sample(other);
                  issue_group_one<E>(ctx, ln, d0, d1, i);
                }))
              break;
          }
          slot = other;
          s += 2;
        }
      }
      if (!atSite) break;  // the tile is computed

      // ---- poll site s with a new generation (or the setter's turn) ----
      siteDone = s;
      int f = fSeen;
      if (isSetter && tid == 0 && f >= 0) {
        const int64_t now = wall_ticks();
        if (s_setter[1] == 0) s_setter[1] = now;
        const long long gBase = s_setter[1];
        const int nextEv = (int)s_setter[0];
        if (nextEv < P().num_events) {
          if (now >= gBase + P().sched[nextEv]) {
            P().set_gt[nextEv] = now;
            s_setter[0] = nextEv + 1;
            set_flag(nextEv + 1);
          }
        } else if (P().stop_after > 0 &&
                   now >= gBase + (P().num_events ? P().sched[P().num_events - 1] : 0) +
                              P().stop_after) {
          set_flag(-1);  // self-terminating run: no host in the loop
        }
      }
      if (f > P().num_events) f = P().num_events;  // never index past the event arrays
      srcKind = AS_IS;
      if (f <= lastSeen) continue;
      const int64_t g = wall_ticks();
      if (tid == 0) {
        if (P().obs_gt) {
          const int obsStride = P().obs_stride > 0 ? P().obs_stride : (int)gridDim.x;
          if (row() < obsStride)
            for (int e = lastSeen; e < f; ++e) P().obs_gt[(size_t)e * obsStride + row()] = g;
        }
        if (startHit) stat(ST_START_SITES, 1);
      }
      const int ev = f - 1;
      lastSeen = f;

      // ---- checkpoint: accumulators and the live stages (live_at) ----
      const int live = live_at(s);
      // `observe`: before the drain, each thread reads its 16 bytes of the
      // last load of the newest stage issued (slot `newest`), and reads them
      // again once every load has landed: a difference means that stage was
      // still in flight when the drain (naive: the save) began. With
      // `naive`, the saved stages are also compared with the landed ring: a
      // difference is a stale checkpoint, which the resumed tile inherits.
      int ckMoved = 0, ckStale = 0;  // uniform: what `observe` found
      // `through`: the slot is read back on another XCD (retreat arm): stores
      // written through (CPOL_SC1), published without an L2 write-back.
      auto save_state = [&](float* dst, bool drain, bool observe, bool through) -> int64_t {
        // the slot of the most recently issued stage
        const int newest = POLL == APK_POLL_ISSUE ? (slot + E::NS - 1) % E::NS : next_slot<E>(slot);
        uint4 before = {0, 0, 0, 0};
        if (observe) before = probe_last_load<E>(ring, newest);
        // drain: every wave's loads landed, then a barrier makes them visible
        // to every thread. naive: no wait and no barrier -- the ring is read
        // as it stands (no wave writes LDS here; only loads may still land).
        if (drain) {
          wait_vmcnt<0>();
          lds_sync();
        }
        const int64_t t0 = wall_ticks();
        if (through) {
          if (P().resume == APK_RESUME_CKPT_FULL)
            Ckpt<E>::template save_ring<CPOL_SC1>(ring, dst, slot, live);
          if (P().resume != APK_RESUME_RESTART) Ckpt<E>::template save_acc<CPOL_SC1>(acc, dst);
        } else {
          if (P().resume == APK_RESUME_CKPT_FULL) Ckpt<E>::save_ring(ring, dst, slot, live);
          if (P().resume != APK_RESUME_RESTART) Ckpt<E>::save_acc(acc, dst);
        }
        if (observe) {
          wait_vmcnt<0>();  // every load landed, every checkpoint store done
          lds_sync();
          const uint4 after = probe_last_load<E>(ring, newest);
          const bool moved = (before.x != after.x) | (before.y != after.y) |
                             (before.z != after.z) | (before.w != after.w);
          const bool stale = !drain && P().resume == APK_RESUME_CKPT_FULL &&
                             Ckpt<E>::ring_differs(ring, dst, slot, live);
          ckMoved = uniform(__syncthreads_or(moved ? 1 : 0) ? 1 : 0);
          ckStale = uniform(__syncthreads_or(stale ? 1 : 0) ? 1 : 0);
          if (tid == 0) {
            stat(ST_INFLIGHT_ALL, (uint64_t)ckMoved);
            stat(ST_STALE_ALL, (uint64_t)ckStale);
            stat(ST_CHECKPOINTS, 1);
          }
        }
        return t0;
      };

      if constexpr (retreatArm) {
        // ---- retreat: hand this block's CU to the kernel on the other stream ----
        // The hardware deals a kernel's workgroups round-robin to the XCDs
        // and their shader engines from wherever its pointers stand, and a
        // workgroup runs only on a CU of its own shader engine: the urgent
        // kernel's R workgroups land in R domains the host cannot name, so
        // free ceil(R / 32) CUs in every (XCD, shader engine) domain.
        // Which blocks retreat at generation f (launch_epoch in the params):
        // of the first grid at f = 1, the ceil(R / 32) blocks per domain that
        // registered first when the grid started; a continuation that follows an
        // earlier generation, all of it -- it holds the CUs the previous
        // generation freed, and it must complete for the next continuation
        // (queued behind it) to start.
        const int role = proto::retreat_role(P().continuation != 0, P().launch_epoch, f);
        const bool mine = mayRetreat;  // by quota: registered among the first at start
        if (P().continuation == 0) mayRetreat = false;  // no later generation is its turn
        if (role == proto::RETREAT_NONE) continue;  // not this block's turn: keep working
        if (role == proto::RETREAT_BY_QUOTA && !mine) continue;
        unsigned t = RQ_NONE;
        if (tid == 0) {
          t = rq_reserve(P().rq_ctl, P().rq_capacity, P().rq_entry);
          if (t == RQ_FULL) {  // the ring holds capacity tickets: declined, keep working
            stat(ST_DECLINED, 1);
            t = RQ_NONE;
          } else if (t & RQ_STUCK) {  // its entry never freed: keep working, report it
            stat(ST_ERRORS, 1);
            t = RQ_NONE;
          } else {
            // counted (the retreats of generation f per domain), no round trip
            __hip_atomic_fetch_add(
                &P().retreat_count[(size_t)ev * APK_RETREAT_DOMAINS + domain()], 1,
                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
        const unsigned tk = bcast(t);
        if (tk == RQ_NONE) continue;  // declined: keep working
        float* dst = P().rq_slots + (size_t)(tk % P().rq_capacity) * Ckpt<E>::SLOT_FLOATS;
        // always drain: nothing may land in LDS after the block exits
        const int64_t tSave = save_state(dst, true, false, true);
        const int rkind = P().resume == APK_RESUME_RESTART ? 0
                          : P().resume == APK_RESUME_CKPT_FULL ? 2 : 1;
        // Every thread's checkpoint stores, written through the L2, have
        // completed: after the barrier, thread 0 publishes the entry (its
        // fields, then their completion, then the sequence number).
        wait_vmcnt<0>();
        lds_sync();
        if (tid == 0) {
          rq_publish(P().rq_entry + (size_t)(tk % P().rq_capacity) * 4, tk, (int)task,
                     rkind > 0 ? s : 0, rkind, domain());
          const int64_t t1 = wall_ticks();
          stat(ST_RETREATS, 1);
          stat(ST_SAVE, (uint64_t)(t1 - tSave));
          if (P().retreat_gt) {
            atomic_min_i64(&P().retreat_gt[2 * (size_t)ev], tSave);
            atomic_max_i64(&P().retreat_gt[2 * (size_t)ev + 1], t1);
          }
        }
        retreated = true;
      } else {
        // ---- cooperative yield: pop the event's mini-queue, checkpoint, serve ----
        const int U = nU();
        const bool drain = !P().naive;
        int64_t tSave;
        if constexpr (POLL == APK_POLL_ISSUE) {
          // Window-forcing order (src/midyield.cu:246-258): checkpoint right
          // after the flag read, before any further wait or atomic, then pop.
          // A block that gets no urgent tile goes on with its state intact.
          tSave = save_state(ckslot(), drain, true, false);
          uidx = U > 0 ? pop_urgent(ev) : U;
          if (uidx >= U) {
            // No urgent tile: resume from the checkpoint just taken all the
            // same, so that every checkpoint taken here is tested on resume.
            if (tid == 0) {
              stat(ST_INFLIGHT, (uint64_t)ckMoved);
              stat(ST_STALE, (uint64_t)ckStale);
            }
            srcKind = P().resume == APK_RESUME_RESTART   ? FRESH
                      : P().resume == APK_RESUME_CKPT_FULL ? FULL
                                                            : ACC;
            src = ckslot();
            if (srcKind == FRESH) s = 0;
            continue;
          }
        } else {
          uidx = U > 0 ? pop_urgent(ev) : U;
          if (uidx >= U) continue;
          tSave = save_state(ckslot(), drain, true, false);
        }
        lds_sync();  // ring reads (checkpoint) done before the urgent tiles overwrite it
        if (tid == 0) {
          const int64_t t1 = wall_ticks();
          s_serve_t1 = t1;
          if (uidx == 0) {
            P().claim[ev] = bid + 1;
            P().claim_site[ev] = s;
            P().u_gt[2 * (size_t)ev] = t1;
          }
          stat(ST_SAVE, (uint64_t)(t1 - tSave));
          stat(ST_INFLIGHT, (uint64_t)ckMoved);
          stat(ST_STALE, (uint64_t)ckStale);
        }
        serving = ev;
        savedTask = task;
        savedStage = s;
        savedKind = P().resume == APK_RESUME_RESTART   ? FRESH
                    : P().resume == APK_RESUME_CKPT_FULL ? FULL
                                                          : ACC;
        yielded = true;
      }
      break;
    }
    if (retreated) break;  // the block exits; its tile waits in the resume queue
    if (yielded) continue;  // the event's urgent tiles first, then this tile again
    if constexpr (kPipe) {
      if (hasTail) E::finish_tail(acc, tail);
    }
    wait_vmcnt<0>();  // the refetches past the tile's end have landed
    lds_sync();       // every wave done with the ring; every sample has landed
    if (POLL != APK_POLL_OFF && lastSlot >= 0) fLatest = uniform(flagring[lastSlot]);

    // ---- epilogue: C tile, fingerprint, exactly-once count ----
    float* C = urgent ? P().Cu + (size_t)serving * (size_t)P().cu_event_stride : P().C;
    unsigned long long* hashDst =
        urgent ? (P().u_hash ? P().u_hash + (size_t)serving * nU() + uidx : nullptr)
               : (P().task_hash ? P().task_hash + task : nullptr);
    const uint64_t hp = store_tile<E>(acc, ring, C, urgent ? P().Nu : P().N, row0, col0,
                                      hashDst != nullptr);
    if (hashDst) {
      const uint64_t h = block_sum_u64(hp, s_red);
      if (tid == 0) *hashDst = h;
    }
    if (ORACLE && tid == 0)
      fetch_add_i32(urgent ? &P().u_exec_count[serving] : &P().exec_count[task], 1);
    if (urgent) uidx = pop_urgent(serving);
    else chunksDone += S / chunkStages;
  }

  // The last exit is the latest one: an atomic max that returns nothing, so
  // a retreating block's CU is not held for a round trip (a count returning
  // "last block?" held it ~0.5 us before the urgent kernel could have it).
  if (P().run_gt && tid == 0) {
    atomic_max_i64(&P().run_gt[1], wall_ticks());
    __hip_atomic_fetch_add(P().exit_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (P().stats && tid == 0) {
    // Added, not stored: relaunches (retreat-arm continuations) may share rows.
    unsigned long long* st = P().stats + (size_t)row() * APK_STATS_PER_BLOCK;
    for (int k = 0; k < APK_STATS_PER_BLOCK; ++k)
      if (s_stats[k])
        __hip_atomic_fetch_add(&st[k], s_stats[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <class E>
static int validate(const apk_yield_params* p, int poll, int oracle, int blocks) {
  APK_REQUIRE(p != nullptr, "persistent_yield: params is NULL");
  APK_REQUIRE(p->A && p->B && p->C && p->next_task, "persistent_yield: NULL GEMM pointer");
  APK_REQUIRE(p->M > 0 && p->N > 0 && p->K > 0 && p->M % E::TM == 0 && p->N % E::TN == 0,
              "persistent_yield: M=%d N=%d K=%d vs %dx%d tiles", p->M, p->N, p->K, E::TM, E::TN);
  APK_REQUIRE(p->k_chunk > 0 && p->k_chunk % E::KS == 0 && p->K % p->k_chunk == 0,
              "persistent_yield: k_chunk=%d must divide K=%d and be a multiple of %d",
              p->k_chunk, p->K, E::KS);
  APK_REQUIRE(p->K % KAlign<E>::value == 0, "persistent_yield: K=%d must be a multiple of %d",
              p->K, KAlign<E>::value);
  APK_REQUIRE((size_t)p->M * p->K * E::ELEM_BYTES < (1ull << 31) &&
                  (size_t)p->K * p->N * E::ELEM_BYTES < (1ull << 31),
              "persistent_yield: operands above 2 GiB are not supported");
  APK_REQUIRE(blocks > 0, "persistent_yield: blocks=%d", blocks);
  APK_REQUIRE(p->num_tasks < (1u << 31), "persistent_yield: num_tasks=%u", p->num_tasks);
  APK_REQUIRE(poll >= APK_POLL_OFF && poll <= APK_POLL_ISSUE, "persistent_yield: poll=%d", poll);
  if (poll == APK_POLL_ISSUE)
    APK_REQUIRE(p->retreat == 0 && p->flag_system == 0,
                "persistent_yield: issue sites are for the cooperative arm on a device flag");
  APK_REQUIRE(p->num_events >= 0, "persistent_yield: num_events < 0");
  if (poll != APK_POLL_OFF) {
    APK_REQUIRE(p->flag != nullptr, "persistent_yield: polling needs a flag");
    APK_REQUIRE(p->flag_copies >= 0 && p->flag_copies <= APK_FLAG_MAX_COPIES,
                "persistent_yield: flag_copies=%d", p->flag_copies);
    if (p->flag_set) APK_REQUIRE(p->sched != nullptr, "persistent_yield: setter without schedule");
    APK_REQUIRE(p->resume >= APK_RESUME_CKPT_FULL && p->resume <= APK_RESUME_RESTART,
                "persistent_yield: resume=%d", p->resume);
    APK_REQUIRE(p->retreat >= 0, "persistent_yield: retreat=%d", p->retreat);
    APK_REQUIRE(p->block_base >= 0 && p->obs_stride >= 0,
                "persistent_yield: block_base=%d obs_stride=%d", p->block_base, p->obs_stride);
    if (p->retreat > 0) {
      APK_REQUIRE(p->num_events > 0 && p->retreat_count && p->rq_ctl && p->rq_entry,
                  "persistent_yield: the retreat arm needs events, retreat_count and a resume "
                  "queue");
      APK_REQUIRE(p->rq_capacity >= 2,
                  "persistent_yield: rq_capacity=%u, the resume ring needs at least 2 entries",
                  p->rq_capacity);
      APK_REQUIRE(p->rq_slots || p->resume == APK_RESUME_RESTART,
                  "persistent_yield: checkpointing retreats need rq_slots");
      APK_REQUIRE(p->Au == nullptr, "persistent_yield: the retreat arm runs no urgent job");
      APK_REQUIRE(p->flag_system == 0, "persistent_yield: the retreat arm polls a device flag");
    } else {
      if (p->num_events > 0)
        APK_REQUIRE(p->set_gt && p->obs_gt && p->claim && p->claim_site && p->u_gt &&
                        p->u_end_max && p->uq_next,
                    "persistent_yield: NULL event array");
      if (p->resume != APK_RESUME_RESTART)
        APK_REQUIRE(p->ckpt != nullptr, "persistent_yield: checkpointing needs ckpt storage");
      APK_REQUIRE(p->block_base == 0, "persistent_yield: block_base is for the retreat arm");
    }
  }
  if (p->Au) {
    APK_REQUIRE(p->Bu && p->Cu && p->Mu > 0 && p->Nu > 0 && p->Ku > 0 &&
                    p->Mu % E::TM == 0 && p->Nu % E::TN == 0 &&
                    p->Ku % KAlign<E>::value == 0,
                "persistent_yield: urgent job %dx%dx%d vs %dx%dx%d granularity", p->Mu,
                p->Nu, p->Ku, E::TM, E::TN, KAlign<E>::value);
  }
  if (oracle)
    APK_REQUIRE(p->exec_count && (p->u_exec_count || !p->Au),
                "persistent_yield: oracle needs count arrays");
  APK_REQUIRE(p->cu_event_stride >= 0 && (p->cu_event_stride == 0 ||
                                          p->cu_event_stride >= (long long)p->Mu * p->Nu),
              "persistent_yield: cu_event_stride=%lld", p->cu_event_stride);
  APK_REQUIRE(!p->run_gt || p->exit_count, "persistent_yield: run_gt needs exit_count");
  return APK_OK;
}

template <class E, int POLL, bool ORACLE, bool SYS, bool RETREAT = false>
static int launch_t(const apk_yield_params* p, int blocks, hipStream_t st) {
  hipLaunchKernelGGL((k_persistent_yield<E, POLL, ORACLE, SYS, RETREAT>), dim3(blocks),
                     dim3(E::THREADS), 0, st, *p);
  APK_LAUNCHED();
  return APK_OK;
}

template <class E, int POLL>
static int launch_p(const apk_yield_params* p, int oracle, int blocks, hipStream_t st) {
  const bool sys = p->flag_system != 0;
  if constexpr (POLL == APK_POLL_ISSUE) {  // cooperative arm, device flag (validated)
    return oracle ? launch_t<E, POLL, true, false>(p, blocks, st)
                  : launch_t<E, POLL, false, false>(p, blocks, st);
  } else {
    if constexpr (POLL != APK_POLL_OFF) {
      if (p->retreat > 0)  // device-memory flag only (validated)
        return oracle ? launch_t<E, POLL, true, false, true>(p, blocks, st)
                      : launch_t<E, POLL, false, false, true>(p, blocks, st);
    }
    if (oracle) return sys ? launch_t<E, POLL, true, true>(p, blocks, st)
                           : launch_t<E, POLL, true, false>(p, blocks, st);
    return sys ? launch_t<E, POLL, false, true>(p, blocks, st)
               : launch_t<E, POLL, false, false>(p, blocks, st);
  }
}

template <class E>
static int launch_e(int poll, int oracle, const apk_yield_params* p, int blocks,
                    hipStream_t st) {
  const int rc = validate<E>(p, poll, oracle, blocks);
  if (rc != APK_OK) return rc;
  switch (poll) {
    case APK_POLL_OFF: return launch_p<E, APK_POLL_OFF>(p, oracle, blocks, st);
    case APK_POLL_CHUNK: return launch_p<E, APK_POLL_CHUNK>(p, oracle, blocks, st);
    case APK_POLL_STAGE: return launch_p<E, APK_POLL_STAGE>(p, oracle, blocks, st);
    default: return launch_p<E, APK_POLL_ISSUE>(p, oracle, blocks, st);
  }
}

}  // namespace apk

extern "C" int apk_persistent_yield(int engine, int poll, int oracle,
                                    const apk_yield_params* params, int blocks,
                                    void* stream) {
  using namespace apk;
  switch (engine) {
    case APK_ENGINE_VALU64:
      return launch_e<EngValu64>(poll, oracle, params, blocks, as_stream(stream));
    case APK_ENGINE_MFMA128:
      return launch_e<EngMfma128>(poll, oracle, params, blocks, as_stream(stream));
    case APK_ENGINE_BF16X256:
      return launch_e<EngBf16x256>(poll, oracle, params, blocks, as_stream(stream));
    case APK_ENGINE_BF16X128:
      return launch_e<EngBf16x128>(poll, oracle, params, blocks, as_stream(stream));
    case APK_ENGINE_BF16X256X128:
      return launch_e<EngBf16x256x128>(poll, oracle, params, blocks, as_stream(stream));
    default:
      set_error("persistent_yield: unknown engine %d", engine);
      return APK_EINVAL;
  }
}

extern "C" long long apk_yield_ckpt_floats(int engine) {
  using namespace apk;
  switch (engine) {
    case APK_ENGINE_VALU64: return Ckpt<EngValu64>::SLOT_FLOATS;
    case APK_ENGINE_MFMA128: return Ckpt<EngMfma128>::SLOT_FLOATS;
    case APK_ENGINE_BF16X256: return Ckpt<EngBf16x256>::SLOT_FLOATS;
    case APK_ENGINE_BF16X128: return Ckpt<EngBf16x128>::SLOT_FLOATS;
    case APK_ENGINE_BF16X256X128: return Ckpt<EngBf16x256x128>::SLOT_FLOATS;
    default: return -1;
  }
}

namespace apk {

// Resident blocks per CU of the instantiation a launch with these settings
// uses (the cooperative, device-flag one; its oracle, host-flag and retreat
// twins differ only off the stage loop), at the engine's block size.
template <class E>
static int yield_occupancy_of(int poll, int* out) {
  int n = 0;
  auto q = [&](auto kern) -> int {
    APK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, E::THREADS, 0));
    return APK_OK;
  };
  int rc;
  switch (poll) {
    case APK_POLL_OFF: rc = q(k_persistent_yield<E, APK_POLL_OFF, false, false, false>); break;
    case APK_POLL_CHUNK: rc = q(k_persistent_yield<E, APK_POLL_CHUNK, false, false, false>); break;
    case APK_POLL_STAGE: rc = q(k_persistent_yield<E, APK_POLL_STAGE, false, false, false>); break;
    case APK_POLL_ISSUE: rc = q(k_persistent_yield<E, APK_POLL_ISSUE, false, false, false>); break;
    default:
      set_error("occupancy: poll %d", poll);
      return APK_EINVAL;
  }
  if (rc != APK_OK) return rc;
  *out = n;
  return APK_OK;
}

}  // namespace apk

extern "C" int apk_persistent_yield_occupancy(int engine, int poll, int* blocks_per_cu) {
  using namespace apk;
  APK_REQUIRE(blocks_per_cu != nullptr, "occupancy: out is NULL");
  switch (engine) {
    case APK_ENGINE_VALU64: return yield_occupancy_of<EngValu64>(poll, blocks_per_cu);
    case APK_ENGINE_MFMA128: return yield_occupancy_of<EngMfma128>(poll, blocks_per_cu);
    case APK_ENGINE_BF16X256: return yield_occupancy_of<EngBf16x256>(poll, blocks_per_cu);
    case APK_ENGINE_BF16X128: return yield_occupancy_of<EngBf16x128>(poll, blocks_per_cu);
    case APK_ENGINE_BF16X256X128:
      return yield_occupancy_of<EngBf16x256x128>(poll, blocks_per_cu);
    default:
      set_error("occupancy: engine %d", engine);
      return APK_EINVAL;
  }
}
