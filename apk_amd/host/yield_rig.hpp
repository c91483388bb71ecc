// yield_rig.hpp -- device buffers and launch of the preemptible persistent
// GEMM (apk_persistent_yield) for the yield and midyield binaries: the
// reference's zero_all / launch / read-back plumbing (src/yield.cu:372-448,
// src/midyield.cu:410-469) gathered in one place.
#pragma once
#include <string>
#include <utility>
#include <vector>

#include "host_common.hpp"

namespace host {

struct RigShape {
  int engine = APK_ENGINE_VALU64;
  int M = 0, N = 0, K = 0, kChunk = 0;
  int Mu = 0, Nu = 0, Ku = 0;  // urgent job (0 = none)
  int blocks = 0;
  int events = 0;              // capacity of the event arrays
  unsigned hashTasks = 0;      // capacity of the per-task fingerprint array (0 = none)
  unsigned oracleTasks = 0;    // capacity of the exactly-once counts (0 = none)
  bool hostFlag = false;       // flag in host-mapped memory (host-set events)
  int flagCopies = 1;          // replicas of the flag, APK_FLAG_STRIDE apart
  bool cuPerEvent = false;     // one urgent output per event (CuAll)
  bool runTimes = false;       // record the run's start / last-exit ticks
  // Retreat arm: resume-queue tickets per job (0 = no retreat arm) and rows
  // of stats kept for relaunched (continuation) blocks after the first
  // `blocks` rows.
  unsigned retreatCap = 0;
  bool retreatSlots = true;  // checkpoint slots for the ring (none: restart only)
  int extraRows = 0;
};

// Per-event timeline of the retreat arm (device ticks).
struct RetreatResult {
  std::vector<long long> setGT;       // flag raised (apk_raise_flag)
  std::vector<long long> retreatGT;   // [2e] earliest checkpoint start, [2e+1] latest exit
  std::vector<int> count;             // [e * 32 + domain] blocks that retreated
  unsigned head = 0, tail = 0;        // resume tickets popped / reserved
  unsigned unclaimed = 0;             // reserved tickets not yet claimed (0 once drained)
  unsigned unreleased = 0;            // reserved tickets not yet released (0 once drained)
  std::vector<int> xcd;               // per reserved ticket: domain (xcd * 4 + se) that retreated
};

struct EventResult {
  std::vector<long long> setGT, obs, uGT;     // ticks
  std::vector<int> claim, site;
  std::vector<unsigned long long> uEnd;
  std::vector<unsigned long long> uHash;
  std::vector<unsigned long long> stats;      // blocks x APK_STATS_PER_BLOCK
};

class YieldRig {
 public:
  YieldRig(const RigShape& s, const std::vector<float>& A, const std::vector<float>& B,
           const std::vector<float>& Au, const std::vector<float>& Bu);
  // Operands as raw bytes in the engine's element type and B layout.
  YieldRig(const RigShape& s, const std::vector<uint8_t>& A, const std::vector<uint8_t>& B,
           const std::vector<uint8_t>& Au, const std::vector<uint8_t>& Bu);
  ~YieldRig();

  const RigShape& shape() const { return s_; }
  int urgentTiles() const { return U_; }
  apk_engine_geometry geo() const { return geo_; }

  // Zero the queue, flag and event arrays (before any launch); fill C / Cu
  // with NaN when nanFill. Synchronizes the device.
  void reset(bool nanFill);
  // (Re)allocate the per-task fingerprint and exactly-once arrays for up to
  // n tasks each (0 = keep the current capacity).
  void reserveTasks(unsigned hashTasks, unsigned oracleTasks);
  // Upload a cumulative schedule (ns) as device ticks.
  void setSchedule(const std::vector<long long>& cumNs, double wallMHz);

  // Launch on `stream`: poll mode, number of tasks, whether block 0 acts as
  // the device setter for `nEvents` events, oracle instantiation.
  void launch(int poll, int pollEvery, int resume, int poison, unsigned numTasks,
              bool devSetter, int nEvents, bool oracle, hipStream_t stream,
              long long stopAfterTicks = 0, int naive = 0);

  // Retreat arm: launch `blocks` workers (rows blockBase.. of stats) that
  // retreat `retreat` blocks per event into the resume queue; continuation
  // = a relaunch joining the running job. runGT (2 ticks) / exitCount may
  // be NULL.
  void launchRetreat(int poll, int pollEvery, int resume, unsigned numTasks, int retreat,
                     int nEvents, bool oracle, int blocks, int blockBase, bool continuation,
                     long long* runGT, unsigned* exitCount, hipStream_t stream,
                     int launchEpoch = 0);
  // Zero the resume queue and the per-event retreat bookkeeping of a job.
  void resetRetreat();
  RetreatResult readRetreat(int nEvents) const;
  long long* dSetGT() const { return dSet_; }

  // Host-mapped flag (host-set mode): relaxed store visible to the GPU.
  void hostSetFlag(int v);

  EventResult readEvents(int nEvents) const;
  std::vector<float> readC() const;
  std::vector<float> readCu() const;           // event 0's (or the shared) output
  std::vector<float> readCuEvent(int e) const; // cuPerEvent
  std::pair<long long, long long> readRunGT() const;  // runTimes: start, last exit
  std::vector<unsigned long long> readTaskHash(unsigned n) const;
  std::vector<int> readExec(unsigned n) const;
  std::vector<int> readUExec(int n) const;

  float* dC() const { return dC_; }
  unsigned* dNextTask() const { return dNext_; }
  int* dFlag() const { return dFlag_; }
  long long* dRunGT() const { return dRunGT_; }
  unsigned* dExitCount() const { return dExit_; }

 private:
  RigShape s_;
  apk_engine_geometry geo_{};
  int U_ = 0;
  float *dA_ = nullptr, *dB_ = nullptr, *dC_ = nullptr;
  float *dAu_ = nullptr, *dBu_ = nullptr, *dCu_ = nullptr;
  unsigned* dNext_ = nullptr;
  int* dFlag_ = nullptr;   // device flag, or device alias of the host flag
  int* hFlag_ = nullptr;   // host-mapped flag (hostFlag mode)
  long long *dSched_ = nullptr, *dSet_ = nullptr, *dObs_ = nullptr, *dUGT_ = nullptr;
  int *dClaim_ = nullptr, *dSite_ = nullptr, *dUq_ = nullptr;
  unsigned long long* dUEnd_ = nullptr;
  float* dCkpt_ = nullptr;
  unsigned long long *dTaskHash_ = nullptr, *dUHash_ = nullptr, *dStats_ = nullptr;
  int *dExec_ = nullptr, *dUExec_ = nullptr;
  long long* dRunGT_ = nullptr;
  unsigned* dExit_ = nullptr;
  int* dRetreatCount_ = nullptr;
  long long* dRetreatGT_ = nullptr;
  unsigned* dRqCtl_ = nullptr;
  int* dRqEntry_ = nullptr;
  float* dRqSlots_ = nullptr;
};

// Per-event summary of an observation matrix (src/yield.cu:889-928).
struct EventRow {
  int event;
  long long setNs, firstNs, lastNs;
  double latUs, spreadUs, e2eUs, b0Us, latX0Us, firstUs;
  int claimer, complete, lastBlock, site;
};
std::vector<EventRow> summarize_events(const EventResult& r, int nEvents, int blocks,
                                       double wallMHz);

// OBS1 matrix dump (src/yield.cu:452-466): int64 {0x3153424f, events,
// blocks}, setGT[events], obs[events*blocks], little-endian, in ns.
void dump_obs1(const char* path, const EventResult& r, int nEvents, int blocks,
               double wallMHz);

}  // namespace host
