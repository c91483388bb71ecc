// protocol_sim -- the scheduler protocol of the persistent kernels on CPU
// threads, for finding queue, claim and resume bugs without a GPU.
//
// One std::thread per block. The work queue, the resume ring and the
// generation rules are the kernels' own code (apk_amd/csrc/protocol.hpp, here
// on host atomics and fences); the block loop around them restates the
// kernels' (apk_amd/csrc/k_yield.hip): take a task (resume ring first in the
// retreat arm, then the work queue), walk its k-stages, poll the generation
// flag every `poll_every` stages, and at a new generation either
//   coop     pop the event's urgent tiles, checkpoint, serve them, restore
//            (src/yield.cu:95-204 is the reference's claim/serve loop), or
//   retreat  (first grid at generation 1: the first `quota` blocks of each
//            domain to start, which alone poll at every site; afterwards the newest
//            continuation) reserve a resume ticket, checkpoint into its slot,
//            publish, exit; a continuation launched after the event resumes
//            the ring's checkpoints.
// A host thread raises the generations at exponential gaps and, in the
// retreat arm, launches one continuation per event (and drains at the end).
//
// The tile "arithmetic" is order-sensitive: a stage folds hash(tile, stage,
// operand word) into a 64-bit accumulator, and a FULL resume computes the
// restored stages from the checkpointed operand words, so a resume at the
// wrong stage, a lost or duplicated stage, or a stale checkpoint changes the
// result. Checked at the end: every task ran to completion exactly once with
// the expected result, every fired event's urgent tiles ran exactly once
// (coop), and the resume ring is empty -- every ticket claimed and released,
// no wait run out (lost, stuck). Retreats the ring declined because it was
// full ("refused") are allowed: the declining block keeps its tile.
//
// --rq-wait-us sets the ring's wait deadlines (the kernels' 20 ms by default).
// --urgent-us: how long the urgent kernel holds the freed CUs before the
// continuation starts (20 us by default).
// --bug plants one mistake, to show that the checks see it:
//   publish-early   (retreat) publish the ticket before writing the slot
//   resume-skip     resume one stage past the checkpointed stage
//   no-release      (retreat) never free a consumed ring entry
//   no-gate         (retreat) reserve without the occupancy gate: take a ticket
//                   first and decline when its entry stays taken past the
//                   deadline (this leaves a hole in the ticket order)
//   double-serve    (coop) serve the urgent tile popped by the previous block again
//
// Exit status 0 when every check passes, 1 otherwise; one summary line.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <chrono>
#include <random>
#include <string>
#include <thread>
#include <vector>

#define APK_PROTO_FN inline
#include "protocol.hpp"

namespace {

// The protocol orders its payload with fences around relaxed flag accesses
// (as the kernels do). ThreadSanitizer cannot model standalone fences, so
// its build (APK_SIM_TSAN) carries the same orderings on the accesses
// themselves -- acquire loads and release stores, which order at least as
// much -- and then reports any plain access to shared state (checkpoint
// slots, results) that no protocol step orders.
#ifdef APK_SIM_TSAN
constexpr int kLoadOrder = __ATOMIC_ACQUIRE, kStoreOrder = __ATOMIC_RELEASE;
#else
constexpr int kLoadOrder = __ATOMIC_RELAXED, kStoreOrder = __ATOMIC_RELAXED;
#endif
struct HostPlat {
  static unsigned fetch_add(unsigned* p, unsigned v) {
    return __atomic_fetch_add(p, v, __ATOMIC_RELAXED);
  }
  static unsigned load(const unsigned* p) { return __atomic_load_n(p, kLoadOrder); }
  static int load(const int* p) { return __atomic_load_n(p, kLoadOrder); }
  static void store(int* p, int v) { __atomic_store_n(p, v, kStoreOrder); }
#ifdef APK_SIM_TSAN
  static void acquire() {}
  static void publish_fence() {}
#else
  static void acquire() { __atomic_thread_fence(__ATOMIC_ACQUIRE); }
  // host payload stores are plain: publishing them takes a release fence
  static void publish_fence() { __atomic_thread_fence(__ATOMIC_RELEASE); }
#endif
  static int64_t ticks() {  // 100 MHz, as the device wall clock
    return std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch()).count() / 10;
  }
  static void pause() { std::this_thread::yield(); }
};
namespace proto = apk::proto;

int64_t now_ns() {
  return std::chrono::duration_cast<std::chrono::nanoseconds>(
             std::chrono::steady_clock::now().time_since_epoch()).count();
}
void spin_ns(int64_t ns) {
  const int64_t end = now_ns() + ns;
  while (now_ns() < end) {
  }
}

uint64_t mix64(uint64_t x) {  // splitmix64 finaliser
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}
// The operand word a stage "loads" and the order-sensitive fold of a stage.
uint64_t operand(unsigned tile, int stage, bool urgent) {
  return mix64(((uint64_t)tile << 32) ^ (uint64_t)stage ^ (urgent ? 0x5a5a000000000000ull : 0));
}
uint64_t fold(uint64_t acc, uint64_t word, int stage) {
  return acc * 6364136223846793005ull + (word ^ (uint64_t)stage);
}
uint64_t expected(unsigned tile, int S, bool urgent) {
  uint64_t acc = 0;
  for (int s = 0; s < S; ++s) acc = fold(acc, operand(tile, s, urgent), s);
  return acc;
}

enum Resume { R_FULL = 2, R_ACC = 1, R_RESTART = 0 };
enum Bug { B_NONE, B_PUBLISH_EARLY, B_RESUME_SKIP, B_NO_RELEASE, B_NO_GATE, B_DOUBLE_SERVE };

struct Config {
  bool retreat = false;
  int blocks = 16, tilesM = 8, tilesN = 8, passes = 4, stages = 16, events = 200;
  double meanGapUs = 300;
  int workNs = 2000, pollEvery = 1, resume = R_FULL, retreatN = 32, cap = 0, urgentTiles = 4;
  int domains = APK_RETREAT_DOMAINS;
  int64_t rqWaitTicks = proto::RQ_WAIT_TICKS;
  int64_t urgentNs = 20000;
  unsigned seed = 21;
  Bug bug = B_NONE;
};

// A checkpoint: accumulator, stage, and (FULL) the operand words of the two
// live stages.
struct Ckpt {
  uint64_t acc;
  int stage;
  uint64_t live[2];
};

struct Sim {
  Config c;
  unsigned numTasks;
  std::vector<unsigned> ctr;                 // work queue counters
  int flag = 0;                              // generation
  std::vector<unsigned> uq;                  // per event: urgent tiles popped
  std::vector<int> uExec;                    // per event x urgent tile: executions
  std::vector<uint64_t> uResult;             // per event x urgent tile
  std::vector<int> exec;                     // per task: completions
  std::vector<uint64_t> result;              // per task
  std::vector<int> retreatCount;             // per event x domain
  std::vector<int> regCount;                 // first grid's blocks per domain, as they start
  unsigned rqCtl[APK_RQ_CTL_WORDS] = {0, 0, 0, 0};
  std::vector<int> rqEntry;                  // cap x 4
  std::vector<Ckpt> rqSlot;                  // cap
  std::atomic<long> retreats{0}, resumed{0}, refused{0}, stuck{0}, lost{0}, yields{0};
  std::atomic<int> running{0};
  // The first grid starts together, as a kernel launch does: its blocks wait
  // for `go`, set once every thread exists (thread creation under the
  // sanitizers takes milliseconds, longer than a whole small job).
  std::atomic<bool> go{false};
  std::atomic<int> fired{0};

  explicit Sim(const Config& cfg) : c(cfg) {
    numTasks = (unsigned)(c.tilesM * c.tilesN * c.passes);
    ctr.assign(16, 0);
    uq.assign(c.events, 0);
    uExec.assign((size_t)c.events * c.urgentTiles, 0);
    uResult.assign((size_t)c.events * c.urgentTiles, 0);
    exec.assign(numTasks, 0);
    result.assign(numTasks, 0);
    retreatCount.assign((size_t)c.events * c.domains, 0);
    regCount.assign(c.domains, 0);
    if (c.cap <= 0) c.cap = 4 * c.retreatN;
    rqEntry.assign((size_t)c.cap * 4, 0);
    for (int i = 0; i < c.cap; ++i) rqEntry[(size_t)i * 4 + 2] = i;  // seq = i: free
    rqSlot.assign(c.cap, Ckpt{});
  }

  // The planted no-gate mistake: the reservation without its occupancy gate
  // (ticket first; a ticket whose entry stays taken past the deadline is
  // declined after it was taken).
  unsigned reserve_ungated() {
    const unsigned t = HostPlat::fetch_add(&rqCtl[1], 1u);
    const int* en = &rqEntry[(size_t)(t % (unsigned)c.cap) * 4];
    const int64_t deadline = HostPlat::ticks() + c.rqWaitTicks;
    while (t >= (unsigned)c.cap && HostPlat::load(&en[2]) != (int)t) {
      if (HostPlat::ticks() > deadline) return proto::RQ_FULL;
      HostPlat::pause();
    }
    HostPlat::fetch_add(&rqCtl[3], 1u);  // keep the occupancy count balanced
    HostPlat::fetch_add(&rqCtl[2], 1u);
    return t;
  }

  // One block: `cont` for a continuation launched after generation `epoch`.
  // The spawner counts the block in `running` before starting its thread.
  void block(int bid, bool cont, int epoch) {
    while (!go.load(std::memory_order_acquire)) std::this_thread::yield();
    std::mt19937 rng(c.seed * 7919u + (unsigned)bid * 131u + (unsigned)epoch);
    const int home = bid & (APK_QUEUE_XCDS - 1);
    const int dom = bid % c.domains;
    const int quota = (c.retreatN + c.domains - 1) / c.domains;
    int lastSeen = 0, chunksDone = 0;  // chunksDone: stage boundaries of completed tasks
    if (cont) lastSeen = proto::first_seen(HostPlat::load(&flag), epoch, c.events);
    // Retreat arm: the first grid's first `quota` blocks of each domain to
    // start retreat at generation 1; a continuation after an earlier
    // generation retreats at the next one. Only such blocks poll at every
    // site; the others at a task's first stage.
    bool mayRetreat = false;
    if (c.retreat)
      mayRetreat = cont ? epoch > 0 && epoch < c.events
                        : __atomic_fetch_add(&regCount[dom], 1, __ATOMIC_RELAXED) < quota;
    proto::TaskQueue<HostPlat> tq(ctr.data(), c.tilesM, c.tilesN, numTasks);
    const unsigned T = (unsigned)(c.tilesM * c.tilesN);
    for (;;) {
      // ---- the next task: resume ring first (retreat arm), else the queue ----
      unsigned task = 0xffffffffu;
      Ckpt ck{};
      int kind = -1;  // -1 new; 0 restart; 1 acc; 2 full
      if (c.retreat) {
        const unsigned q = proto::rq_pop<HostPlat>(rqCtl);
        if (q != proto::RQ_NONE) {
          int* en = &rqEntry[(size_t)(q % (unsigned)c.cap) * 4];
          const int ready = proto::rq_wait_ready<HostPlat>(en, q, c.rqWaitTicks);
          if (ready == 0) {
            lost.fetch_add(1);
            continue;
          }
          task = (unsigned)en[0];
          kind = ready - 1;
          if (kind > 0) ck = rqSlot[q % (unsigned)c.cap];
          ck.stage = en[1];
          if (c.bug != B_NO_RELEASE) proto::rq_release<HostPlat>(rqCtl, en, q, (unsigned)c.cap);
          resumed.fetch_add(1);
        }
      }
      if (task == 0xffffffffu) task = tq.pop(home);
      if (task >= numTasks) break;
      const unsigned tile = task % T;
      const int S = c.stages;

      // ---- the stage loop with its poll sites ----
      uint64_t acc = 0;
      int s = 0;
      uint64_t carried[2] = {0, 0};  // operand words restored with a FULL checkpoint
      int nCarried = 0;
      auto enter = [&](const Ckpt& k, int kd) {
        if (kd == R_RESTART) {
          acc = 0;
          s = 0;
          nCarried = 0;
          return;
        }
        acc = k.acc;
        s = k.stage + (c.bug == B_RESUME_SKIP ? 1 : 0);
        nCarried = 0;
        if (kd == R_FULL) {
          carried[0] = k.live[0];
          carried[1] = k.live[1];
          nCarried = 2;
        }
      };
      if (kind >= 0) enter(ck, kind);
      bool retreated = false;
      while (s < S) {
        // every poll_every-th boundary passed (a block that can no longer
        // retreat: a task's first stage)
        if ((!c.retreat || mayRetreat) ? (chunksDone + s) % c.pollEvery == 0 : s == 0) {
          int f = HostPlat::load(&flag);
          if (f > c.events) f = c.events;
          if (f > lastSeen) {
            const int ev = f - 1;
            lastSeen = f;
            // the live stages s, s+1: restored words not yet consumed, else loaded
            Ckpt mine{acc, s, {operand(tile, s, false), s + 1 < S ? operand(tile, s + 1, false) : 0}};
            if (nCarried == 2) {
              mine.live[0] = carried[0];
              mine.live[1] = carried[1];
            } else if (nCarried == 1) {
              mine.live[0] = carried[1];
            }
            if (c.retreat) {
              const int role = proto::retreat_role(cont, epoch, f);
              const bool chosen = mayRetreat;
              if (!cont) mayRetreat = false;
              if (role == proto::RETREAT_ALL || (role == proto::RETREAT_BY_QUOTA && chosen)) {
                const unsigned t = c.bug == B_NO_GATE
                                       ? reserve_ungated()
                                       : proto::rq_reserve<HostPlat>(rqCtl, (unsigned)c.cap,
                                                                     rqEntry.data(), c.rqWaitTicks);
                if (t == proto::RQ_FULL) {
                  refused.fetch_add(1);
                } else if (t & proto::RQ_STUCK) {
                  stuck.fetch_add(1);
                } else {
                  int* en = &rqEntry[(size_t)(t % (unsigned)c.cap) * 4];
                  const int rk = c.resume;
                  if (c.bug == B_PUBLISH_EARLY) {
                    proto::rq_publish<HostPlat>(en, t, (int)task, rk > 0 ? s : 0, rk, dom);
                    spin_ns(20000);
                    rqSlot[t % (unsigned)c.cap] = mine;
                  } else {
                    rqSlot[t % (unsigned)c.cap] = mine;
                    proto::rq_publish<HostPlat>(en, t, (int)task, rk > 0 ? s : 0, rk, dom);
                  }
                  __atomic_fetch_add(&retreatCount[(size_t)ev * c.domains + dom], 1,
                                     __ATOMIC_RELAXED);
                  retreats.fetch_add(1);
                  retreated = true;
                  break;
                }
              }
            } else {
              // cooperative: pop the event's urgent tiles, serve, resume
              unsigned u = __atomic_fetch_add(&uq[ev], 1u, __ATOMIC_RELAXED);
              if ((int)u < c.urgentTiles) {
                const Ckpt saved = mine;
                unsigned prev = u;
                while ((int)u < c.urgentTiles) {
                  const uint64_t r = expected(u + 1000u * (unsigned)ev, 4, true);
                  __atomic_fetch_add(&uExec[(size_t)ev * c.urgentTiles + u], 1, __ATOMIC_RELAXED);
                  uResult[(size_t)ev * c.urgentTiles + u] = r;
                  prev = u;
                  u = __atomic_fetch_add(&uq[ev], 1u, __ATOMIC_RELAXED);
                }
                if (c.bug == B_DOUBLE_SERVE && prev + 1 < (unsigned)c.urgentTiles)
                  __atomic_fetch_add(&uExec[(size_t)ev * c.urgentTiles + prev + 1], 1,
                                     __ATOMIC_RELAXED);
                yields.fetch_add(1);
                enter(saved, c.resume);
              }
            }
          }
        }
        // compute stage s: its operand word comes from the restored ring for
        // the first two stages after a FULL resume, else it is "loaded"
        uint64_t w = operand(tile, s, false);
        if (nCarried) {
          w = carried[2 - nCarried];
          --nCarried;
        }
        acc = fold(acc, w, s);
        if (c.workNs) spin_ns(c.workNs + (int)(rng() % (unsigned)(c.workNs / 2 + 1)));
        ++s;
      }
      if (retreated) break;  // the block exits: its CUs go to the urgent kernel
      chunksDone += S;
      __atomic_fetch_add(&exec[task], 1, __ATOMIC_RELAXED);
      result[task] = acc;
    }
    running.fetch_sub(1);
  }
};

Bug parse_bug(const std::string& s) {
  if (s == "publish-early") return B_PUBLISH_EARLY;
  if (s == "resume-skip") return B_RESUME_SKIP;
  if (s == "no-release") return B_NO_RELEASE;
  if (s == "no-gate") return B_NO_GATE;
  if (s == "double-serve") return B_DOUBLE_SERVE;
  return B_NONE;
}

}  // namespace

int main(int argc, char** argv) {
  Config c;
  std::string bug = "none";
  for (int i = 1; i + 1 < argc; i += 2) {
    const std::string k = argv[i];
    const char* v = argv[i + 1];
    if (k == "--arm") c.retreat = std::string(v) == "retreat";
    else if (k == "--blocks") c.blocks = atoi(v);
    else if (k == "--tiles-m") c.tilesM = atoi(v);
    else if (k == "--tiles-n") c.tilesN = atoi(v);
    else if (k == "--passes") c.passes = atoi(v);
    else if (k == "--stages") c.stages = atoi(v);
    else if (k == "--events") c.events = atoi(v);
    else if (k == "--mean-gap-us") c.meanGapUs = atof(v);
    else if (k == "--work-ns") c.workNs = atoi(v);
    else if (k == "--poll-every") c.pollEvery = atoi(v);
    else if (k == "--resume")
      c.resume = std::string(v) == "acc" ? R_ACC : std::string(v) == "restart" ? R_RESTART : R_FULL;
    else if (k == "--retreat") c.retreatN = atoi(v);
    else if (k == "--cap") c.cap = atoi(v);
    else if (k == "--urgent-tiles") c.urgentTiles = atoi(v);
    else if (k == "--domains") c.domains = atoi(v);
    else if (k == "--seed") c.seed = (unsigned)atoi(v);
    else if (k == "--rq-wait-us") c.rqWaitTicks = (int64_t)(atof(v) * 100.0);
    else if (k == "--urgent-us") c.urgentNs = (int64_t)(atof(v) * 1000.0);
    else if (k == "--bug") bug = v;
    else {
      fprintf(stderr, "unknown option %s\n", k.c_str());
      return 2;
    }
  }
  c.bug = parse_bug(bug);
  if (c.blocks < 1 || c.stages < 2 || c.events < 0 || c.pollEvery < 1 || c.domains < 1 ||
      c.domains > APK_RETREAT_DOMAINS || c.urgentTiles < 1 || c.tilesM < 1 || c.tilesN < 1 ||
      c.passes < 1 || (c.cap != 0 && c.cap < 2) || c.rqWaitTicks < 0 || c.urgentNs < 0) {
    fprintf(stderr, "bad configuration\n");
    return 2;
  }
  Sim sim(c);
  std::vector<std::thread> threads;
  threads.reserve((size_t)c.blocks * 2 + (size_t)c.events * 2);
  auto spawn = [&](int bid, bool cont, int epoch) {
    sim.running.fetch_add(1);
    threads.emplace_back(&Sim::block, &sim, bid, cont, epoch);
  };
  for (int b = 0; b < c.blocks; ++b) spawn(b, false, 0);
  sim.go.store(true, std::memory_order_release);

  // Host: raise the generations at exponential gaps while blocks still run;
  // retreat arm: after each, the "urgent kernel" (a short wait) and the
  // continuation that brings back as many blocks as the generation freed.
  // On the GPU the next flag is raised on the urgent stream behind the urgent
  // GEMM, which cannot start before a block has retreated (or the job ended):
  // the host here likewise waits for the generation's first retreat (or
  // refusal), up to the ring's 20 ms deadline, so that two generations never
  // land together on a grid that has not reached a site yet.
  std::mt19937 rng(c.seed);
  std::exponential_distribution<double> gap(1.0 / std::max(1.0, c.meanGapUs * 1000.0));
  int nextBid = c.blocks;
  long prevRetreats = 0;
  for (int e = 0; e < c.events; ++e) {
    spin_ns((int64_t)gap(rng));
    if (sim.running.load() == 0) break;
    __atomic_store_n(&sim.flag, e + 1, __ATOMIC_RELAXED);
    sim.fired.fetch_add(1);
    if (c.retreat) {
      const long r0 = sim.retreats.load(), f0 = sim.refused.load();
      const int64_t t0 = now_ns();
      while (sim.retreats.load() == r0 && sim.refused.load() == f0 && sim.running.load() > 0 &&
             now_ns() - t0 < 20000000)
        std::this_thread::yield();
      spin_ns(c.urgentNs);  // the urgent kernel on the freed CUs
      const long r = sim.retreats.load();
      const int n = (int)(r - prevRetreats);
      prevRetreats = r;
      for (int i = 0; i < n; ++i) spawn(nextBid++, true, e + 1);
    }
  }
  // Late drains (retreat arm): checkpoints published after every worker left.
  for (auto& t : threads) t.join();
  threads.clear();
  int drains = 0;
  while (c.retreat && HostPlat::load(&sim.rqCtl[1]) > HostPlat::load(&sim.rqCtl[0]) &&
         drains < 4) {
    ++drains;
    for (int b = 0; b < c.blocks; ++b) spawn(nextBid++, true, c.events);
    for (auto& t : threads) t.join();
    threads.clear();
  }

  // ---- checks ----
  long dup = 0, miss = 0, wrong = 0;
  const unsigned T = (unsigned)(c.tilesM * c.tilesN);
  for (unsigned t = 0; t < sim.numTasks; ++t) {
    if (sim.exec[t] == 0) ++miss;
    if (sim.exec[t] > 1) ++dup;
    if (sim.exec[t] >= 1 && sim.result[t] != expected(t % T, c.stages, false)) ++wrong;
  }
  long uBad = 0, uUnclaimed = 0;
  const int fired = sim.fired.load();
  if (!c.retreat)
    for (int e = 0; e < fired; ++e) {
      const bool any = sim.uq[e] > 0;
      if (!any) {
        ++uUnclaimed;  // every block had finished before it saw the event
        continue;
      }
      for (int u = 0; u < c.urgentTiles; ++u) {
        const size_t i = (size_t)e * c.urgentTiles + u;
        if (sim.uExec[i] != 1 ||
            sim.uResult[i] != expected((unsigned)u + 1000u * (unsigned)e, 4, true))
          ++uBad;
      }
    }
  const long left = (long)(HostPlat::load(&sim.rqCtl[1]) - HostPlat::load(&sim.rqCtl[0]));
  const long unclaimed = (int)HostPlat::load(&sim.rqCtl[2]);
  const long unreleased = (int)HostPlat::load(&sim.rqCtl[3]);
  const bool ok = dup == 0 && miss == 0 && wrong == 0 && uBad == 0 && left == 0 &&
                  unclaimed == 0 && unreleased == 0 && sim.lost.load() == 0 &&
                  sim.stuck.load() == 0 &&
                  (!c.retreat || sim.resumed.load() == sim.retreats.load());
  printf("%s arm=%s blocks=%d tasks=%u stages=%d resume=%s events fired=%d | tasks: dup %ld "
         "miss %ld wrong %ld | %s %ld | resumed %ld | ring left %ld lost %ld refused %ld "
         "stuck %ld unreleased %ld unclaimed tickets %ld | drains %d | urgent bad %ld "
         "unclaimed %ld | bug=%s\n",
         ok ? "PASS" : "FAIL", c.retreat ? "retreat" : "coop", c.blocks, sim.numTasks, c.stages,
         c.resume == R_FULL ? "full" : c.resume == R_ACC ? "acc" : "restart", fired, dup, miss,
         wrong, c.retreat ? "retreats" : "yields",
         c.retreat ? sim.retreats.load() : sim.yields.load(), sim.resumed.load(), left,
         sim.lost.load(), sim.refused.load(), sim.stuck.load(), unreleased, unclaimed, drains,
         uBad, uUnclaimed, bug.c_str());
  return ok ? 0 : 1;
}
