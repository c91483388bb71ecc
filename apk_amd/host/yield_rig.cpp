// yield_rig.cpp -- see yield_rig.hpp.
#include "yield_rig.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace host {

template <class T>
static T* dalloc(size_t n) {
  T* p = nullptr;
  if (n == 0) return nullptr;
  HIP_CHECK(hipMalloc(&p, n * sizeof(T)));
  return p;
}

YieldRig::YieldRig(const RigShape& s, const std::vector<float>& A,
                   const std::vector<float>& B, const std::vector<float>& Au,
                   const std::vector<float>& Bu)
    : YieldRig(s, as_bytes(A), as_bytes(B), as_bytes(Au), as_bytes(Bu)) {}

YieldRig::YieldRig(const RigShape& s, const std::vector<uint8_t>& A,
                   const std::vector<uint8_t>& B, const std::vector<uint8_t>& Au,
                   const std::vector<uint8_t>& Bu)
    : s_(s) {
  APK_CHECK(apk_engine_geometry_of(s.engine, &geo_));
  U_ = (s.Mu > 0 && s.Nu > 0) ? (s.Mu / geo_.tile_m) * (s.Nu / geo_.tile_n) : 0;
  const int E = s.events > 0 ? s.events : 1;
  dA_ = (float*)dalloc<uint8_t>(A.size());
  dB_ = (float*)dalloc<uint8_t>(B.size());
  dC_ = dalloc<float>((size_t)s.M * s.N);
  HIP_CHECK(hipMemcpy(dA_, A.data(), A.size(), hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(dB_, B.data(), B.size(), hipMemcpyHostToDevice));
  if (U_ > 0) {
    dAu_ = (float*)dalloc<uint8_t>(Au.size());
    dBu_ = (float*)dalloc<uint8_t>(Bu.size());
    dCu_ = dalloc<float>((size_t)s.Mu * s.Nu * (s.cuPerEvent ? E : 1));
    HIP_CHECK(hipMemcpy(dAu_, Au.data(), Au.size(), hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(dBu_, Bu.data(), Bu.size(), hipMemcpyHostToDevice));
  }
  dNext_ = dalloc<unsigned>(APK_QUEUE_WORDS);
  const size_t flagBytes = (size_t)APK_FLAG_MAX_COPIES * APK_FLAG_STRIDE;
  if (s.hostFlag) {
    HIP_CHECK(hipHostMalloc((void**)&hFlag_, flagBytes, hipHostMallocCoherent | hipHostMallocMapped));
    memset(hFlag_, 0, flagBytes);
    HIP_CHECK(hipHostGetDevicePointer((void**)&dFlag_, hFlag_, 0));
  } else {
    dFlag_ = dalloc<int>(flagBytes / 4);
  }
  dSched_ = dalloc<long long>(E);
  dSet_ = dalloc<long long>(E);
  dObs_ = dalloc<long long>((size_t)E * s.blocks);
  dUGT_ = dalloc<long long>(2 * (size_t)E);
  dClaim_ = dalloc<int>(E);
  dSite_ = dalloc<int>(E);
  dUq_ = dalloc<int>(E);
  dUEnd_ = dalloc<unsigned long long>(E);
  dCkpt_ = dalloc<float>((size_t)s.blocks * apk_yield_ckpt_floats(s.engine));
  if (s.hashTasks) dTaskHash_ = dalloc<unsigned long long>(s.hashTasks);
  if (U_ > 0) dUHash_ = dalloc<unsigned long long>((size_t)E * U_);
  dStats_ = dalloc<unsigned long long>((size_t)(s.blocks + s.extraRows) * APK_STATS_PER_BLOCK);
  if (s.retreatCap) {
    dRetreatCount_ = dalloc<int>((size_t)(E + 1) * APK_RETREAT_DOMAINS);  // + registrations
    dRetreatGT_ = dalloc<long long>(2 * (size_t)E);
    dRqCtl_ = dalloc<unsigned>(APK_RQ_CTL_WORDS);
    dRqEntry_ = dalloc<int>((size_t)s.retreatCap * 4);
    if (s.retreatSlots)
      dRqSlots_ = dalloc<float>((size_t)s.retreatCap * apk_yield_ckpt_floats(s.engine));
  }
  if (s.oracleTasks) {
    dExec_ = dalloc<int>(s.oracleTasks);
    dUExec_ = dalloc<int>(E);
  }
  if (s.runTimes) {
    dRunGT_ = dalloc<long long>(2);
    dExit_ = dalloc<unsigned>(1);
  }
}

YieldRig::~YieldRig() {
  // Process-lifetime buffers, as the reference (freed at exit).
  if (hFlag_) (void)hipHostFree(hFlag_);
}

void YieldRig::reset(bool nanFill) {
  const int E = s_.events > 0 ? s_.events : 1;
  HIP_CHECK(hipDeviceSynchronize());
  HIP_CHECK(hipMemset(dNext_, 0, APK_QUEUE_WORDS * sizeof(unsigned)));
  if (hFlag_) hostSetFlag(0);
  else HIP_CHECK(hipMemset(dFlag_, 0, (size_t)APK_FLAG_MAX_COPIES * APK_FLAG_STRIDE));
  HIP_CHECK(hipMemset(dSet_, 0, E * sizeof(long long)));
  HIP_CHECK(hipMemset(dObs_, 0, (size_t)E * s_.blocks * sizeof(long long)));
  HIP_CHECK(hipMemset(dUGT_, 0, 2 * (size_t)E * sizeof(long long)));
  HIP_CHECK(hipMemset(dClaim_, 0, E * sizeof(int)));
  HIP_CHECK(hipMemset(dSite_, 0xFF, E * sizeof(int)));
  HIP_CHECK(hipMemset(dUq_, 0, E * sizeof(int)));
  HIP_CHECK(hipMemset(dUEnd_, 0, E * sizeof(unsigned long long)));
  HIP_CHECK(hipMemset(dStats_, 0, (size_t)(s_.blocks + s_.extraRows) * APK_STATS_PER_BLOCK * 8));
  if (s_.retreatCap) resetRetreat();
  if (dTaskHash_) HIP_CHECK(hipMemset(dTaskHash_, 0, (size_t)s_.hashTasks * 8));
  if (dUHash_) HIP_CHECK(hipMemset(dUHash_, 0, (size_t)E * U_ * 8));
  if (dExec_) {
    HIP_CHECK(hipMemset(dExec_, 0, (size_t)s_.oracleTasks * sizeof(int)));
    HIP_CHECK(hipMemset(dUExec_, 0, E * sizeof(int)));
  }
  if (dRunGT_) {
    HIP_CHECK(hipMemset(dRunGT_, 0, 2 * sizeof(long long)));
    HIP_CHECK(hipMemset(dExit_, 0, sizeof(unsigned)));
  }
  if (nanFill) {
    HIP_CHECK(hipMemset(dC_, 0xFF, (size_t)s_.M * s_.N * 4));
    if (dCu_)
      HIP_CHECK(hipMemset(dCu_, 0xFF, (size_t)s_.Mu * s_.Nu * 4 * (s_.cuPerEvent ? E : 1)));
  }
  // Null-stream fills do not order against non-blocking streams
  // (src/yield.cu:681-684): hard sync before any launch.
  HIP_CHECK(hipDeviceSynchronize());
}

void YieldRig::reserveTasks(unsigned hashTasks, unsigned oracleTasks) {
  HIP_CHECK(hipDeviceSynchronize());
  if (hashTasks > s_.hashTasks) {
    if (dTaskHash_) HIP_CHECK(hipFree(dTaskHash_));
    dTaskHash_ = dalloc<unsigned long long>(hashTasks);
    s_.hashTasks = hashTasks;
  }
  if (oracleTasks > s_.oracleTasks) {
    if (dExec_) HIP_CHECK(hipFree(dExec_));
    dExec_ = dalloc<int>(oracleTasks);
    if (!dUExec_) dUExec_ = dalloc<int>(s_.events > 0 ? s_.events : 1);
    s_.oracleTasks = oracleTasks;
  }
}

void YieldRig::setSchedule(const std::vector<long long>& cumNs, double wallMHz) {
  std::vector<long long> t(cumNs.size());
  for (size_t i = 0; i < cumNs.size(); ++i)
    t[i] = (long long)std::llround(cumNs[i] * wallMHz / 1000.0);
  const size_t n = std::min<size_t>(t.size(), s_.events > 0 ? s_.events : 1);
  HIP_CHECK(hipMemcpy(dSched_, t.data(), n * sizeof(long long), hipMemcpyHostToDevice));
}

void YieldRig::launch(int poll, int pollEvery, int resume, int poison, unsigned numTasks,
                      bool devSetter, int nEvents, bool oracle, hipStream_t stream,
                      long long stopAfterTicks, int naive) {
  apk_yield_params p;
  memset(&p, 0, sizeof p);
  p.A = dA_;
  p.B = dB_;
  p.C = dC_;
  p.M = s_.M;
  p.N = s_.N;
  p.K = s_.K;
  p.k_chunk = s_.kChunk;
  p.num_tasks = numTasks;
  p.next_task = dNext_;
  if (U_ > 0) {
    p.Au = dAu_;
    p.Bu = dBu_;
    p.Cu = dCu_;
    p.Mu = s_.Mu;
    p.Nu = s_.Nu;
    p.Ku = s_.Ku;
  }
  p.uq_next = dUq_;
  p.flag = dFlag_;
  p.flag_copies = s_.flagCopies;
  p.flag_system = hFlag_ ? 1 : 0;
  p.flag_set = devSetter ? dFlag_ : nullptr;
  p.sched = devSetter ? dSched_ : nullptr;
  p.num_events = nEvents;
  p.stop_after = devSetter ? stopAfterTicks : 0;
  p.poll_every = pollEvery;
  p.set_gt = dSet_;
  p.obs_gt = dObs_;
  p.claim = dClaim_;
  p.claim_site = dSite_;
  p.u_gt = dUGT_;
  p.u_end_max = dUEnd_;
  p.resume = resume;
  p.ckpt = dCkpt_;
  p.poison = poison;
  p.task_hash = (dTaskHash_ && numTasks <= s_.hashTasks) ? dTaskHash_ : nullptr;
  p.u_hash = dUHash_;
  p.stats = dStats_;
  p.cu_event_stride = s_.cuPerEvent ? (long long)s_.Mu * s_.Nu : 0;
  p.naive = naive;
  p.run_gt = dRunGT_;
  p.exit_count = dExit_;
  if (oracle) {
    if (!dExec_ || numTasks > s_.oracleTasks) {
      fprintf(stderr, "oracle launch needs %u task counters (have %u)\n", numTasks,
              s_.oracleTasks);
      exit(1);
    }
    p.exec_count = dExec_;
    p.u_exec_count = dUExec_;
  }
  APK_CHECK(apk_persistent_yield(s_.engine, poll, oracle ? 1 : 0, &p, s_.blocks, stream));
}

void YieldRig::resetRetreat() {
  const int E = s_.events > 0 ? s_.events : 1;
  HIP_CHECK(hipMemset(dRetreatCount_, 0, (size_t)(E + 1) * APK_RETREAT_DOMAINS * sizeof(int)));
  std::vector<long long> gt(2 * (size_t)E, 0);
  for (int e = 0; e < E; ++e) gt[2 * (size_t)e] = INT64_MAX;
  HIP_CHECK(hipMemcpy(dRetreatGT_, gt.data(), gt.size() * 8, hipMemcpyHostToDevice));
  HIP_CHECK(hipMemset(dRqCtl_, 0, APK_RQ_CTL_WORDS * sizeof(unsigned)));
  // entry i = {task, stage, seq, kind << 8 | domain}; seq = i: free for ticket i
  std::vector<int> en((size_t)s_.retreatCap * 4, 0);
  for (unsigned i = 0; i < s_.retreatCap; ++i) en[(size_t)i * 4 + 2] = (int)i;
  HIP_CHECK(hipMemcpy(dRqEntry_, en.data(), en.size() * sizeof(int), hipMemcpyHostToDevice));
  HIP_CHECK(hipMemset(dSet_, 0, E * sizeof(long long)));
}

void YieldRig::launchRetreat(int poll, int pollEvery, int resume, unsigned numTasks,
                             int retreat, int nEvents, bool oracle, int blocks, int blockBase,
                             bool continuation, long long* runGT, unsigned* exitCount,
                             hipStream_t stream, int launchEpoch) {
  if (!s_.retreatCap || blockBase + blocks > s_.blocks + s_.extraRows) {
    fprintf(stderr, "launchRetreat: no resume queue, or stats rows %d..%d beyond %d\n",
            blockBase, blockBase + blocks, s_.blocks + s_.extraRows);
    exit(1);
  }
  apk_yield_params p;
  memset(&p, 0, sizeof p);
  p.A = dA_;
  p.B = dB_;
  p.C = dC_;
  p.M = s_.M;
  p.N = s_.N;
  p.K = s_.K;
  p.k_chunk = s_.kChunk;
  p.num_tasks = numTasks;
  p.next_task = dNext_;
  p.flag = dFlag_;
  p.flag_copies = s_.flagCopies;
  p.flag_system = hFlag_ ? 1 : 0;
  p.num_events = nEvents;
  p.poll_every = pollEvery;
  p.resume = resume;
  p.task_hash = (dTaskHash_ && numTasks <= s_.hashTasks) ? dTaskHash_ : nullptr;
  p.stats = dStats_;
  p.run_gt = runGT;
  p.exit_count = exitCount;
  if (oracle) {
    if (!dExec_ || numTasks > s_.oracleTasks) {
      fprintf(stderr, "oracle launch needs %u task counters (have %u)\n", numTasks,
              s_.oracleTasks);
      exit(1);
    }
    p.exec_count = dExec_;
  }
  p.retreat = retreat;
  p.retreat_count = dRetreatCount_;
  p.retreat_gt = dRetreatGT_;
  p.rq_ctl = dRqCtl_;
  p.rq_entry = dRqEntry_;
  p.rq_slots = dRqSlots_;
  p.rq_capacity = s_.retreatCap;
  p.continuation = continuation ? 1 : 0;
  p.launch_epoch = launchEpoch;
  p.block_base = blockBase;
  APK_CHECK(apk_persistent_yield(s_.engine, poll, oracle ? 1 : 0, &p, blocks, stream));
}

RetreatResult YieldRig::readRetreat(int nEvents) const {
  RetreatResult r;
  const int n = std::max(nEvents, 1);
  r.setGT.resize(n);
  r.retreatGT.resize(2 * (size_t)n);
  r.count.resize((size_t)n * APK_RETREAT_DOMAINS);
  HIP_CHECK(hipMemcpy(r.setGT.data(), dSet_, n * 8, hipMemcpyDeviceToHost));
  HIP_CHECK(hipMemcpy(r.retreatGT.data(), dRetreatGT_, 2 * (size_t)n * 8, hipMemcpyDeviceToHost));
  HIP_CHECK(hipMemcpy(r.count.data(), dRetreatCount_, r.count.size() * sizeof(int),
                      hipMemcpyDeviceToHost));
  unsigned ctl[APK_RQ_CTL_WORDS];
  HIP_CHECK(hipMemcpy(ctl, dRqCtl_, sizeof ctl, hipMemcpyDeviceToHost));
  r.head = ctl[0];
  r.tail = ctl[1];
  r.unclaimed = ctl[2];
  r.unreleased = ctl[3];
  // the domains of the last min(tail, capacity) retreats, oldest first
  const unsigned n4 = std::min(r.tail, s_.retreatCap);
  std::vector<int> en((size_t)s_.retreatCap * 4);
  HIP_CHECK(hipMemcpy(en.data(), dRqEntry_, en.size() * sizeof(int), hipMemcpyDeviceToHost));
  for (unsigned t = r.tail - n4; t < r.tail; ++t)
    r.xcd.push_back(en[(size_t)(t % s_.retreatCap) * 4 + 3] & 0xff);
  return r;
}

void YieldRig::hostSetFlag(int v) {
  if (!hFlag_) {
    fprintf(stderr, "hostSetFlag without a host-mapped flag\n");
    exit(1);
  }
  for (int c = 0; c < std::max(1, s_.flagCopies); ++c)
    __atomic_store_n((int*)((char*)hFlag_ + (size_t)c * APK_FLAG_STRIDE), v, __ATOMIC_SEQ_CST);
}

template <class T>
static std::vector<T> d2h(const T* d, size_t n) {
  std::vector<T> h(n);
  if (n && d) HIP_CHECK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
  return h;
}

EventResult YieldRig::readEvents(int nEvents) const {
  EventResult r;
  const size_t E = nEvents > 0 ? nEvents : 0;
  r.setGT = d2h(dSet_, E);
  r.obs = d2h(dObs_, E * s_.blocks);
  r.uGT = d2h(dUGT_, 2 * E);
  r.claim = d2h(dClaim_, E);
  r.site = d2h(dSite_, E);
  r.uEnd = d2h(dUEnd_, E);
  if (dUHash_) r.uHash = d2h(dUHash_, E * U_);
  r.stats = d2h(dStats_, (size_t)(s_.blocks + s_.extraRows) * APK_STATS_PER_BLOCK);
  return r;
}

std::vector<float> YieldRig::readC() const { return d2h(dC_, (size_t)s_.M * s_.N); }
std::vector<float> YieldRig::readCu() const {
  return d2h(dCu_, dCu_ ? (size_t)s_.Mu * s_.Nu : 0);
}
std::vector<float> YieldRig::readCuEvent(int e) const {
  const size_t n = (size_t)s_.Mu * s_.Nu;
  std::vector<float> h(dCu_ ? n : 0);
  if (dCu_)
    HIP_CHECK(hipMemcpy(h.data(), dCu_ + (s_.cuPerEvent ? (size_t)e * n : 0), n * 4,
                        hipMemcpyDeviceToHost));
  return h;
}
std::pair<long long, long long> YieldRig::readRunGT() const {
  long long t[2] = {0, 0};
  if (dRunGT_) HIP_CHECK(hipMemcpy(t, dRunGT_, sizeof t, hipMemcpyDeviceToHost));
  return {t[0], t[1]};
}
std::vector<unsigned long long> YieldRig::readTaskHash(unsigned n) const {
  return d2h(dTaskHash_, dTaskHash_ ? std::min(n, s_.hashTasks) : 0);
}
std::vector<int> YieldRig::readExec(unsigned n) const {
  return d2h(dExec_, dExec_ ? std::min(n, s_.oracleTasks) : 0);
}
std::vector<int> YieldRig::readUExec(int n) const { return d2h(dUExec_, dUExec_ ? n : 0); }

std::vector<EventRow> summarize_events(const EventResult& r, int nEvents, int blocks,
                                       double wallMHz) {
  const double nsPerTick = 1000.0 / wallMHz;
  std::vector<EventRow> out;
  for (int e = 0; e < nEvents; ++e) {
    EventRow row{};
    row.event = e;
    const long long set = r.setGT[e];
    row.setNs = (long long)(set * nsPerTick);
    long long lo = 0, hi = 0, hiX0 = 0;
    int seen = 0, lastBlock = -1;
    for (int b = 0; b < blocks; ++b) {
      const long long o = r.obs[(size_t)e * blocks + b];
      if (o == 0) continue;
      ++seen;
      lo = (lo == 0 || o < lo) ? o : lo;
      if (o > hi) {
        hi = o;
        lastBlock = b;
      }
      if (b > 0 && o > hiX0) hiX0 = o;
    }
    row.firstNs = (long long)(lo * nsPerTick);
    row.lastNs = (long long)(hi * nsPerTick);
    row.complete = seen == blocks;
    row.lastBlock = lastBlock;
    row.latUs = (hi - set) * nsPerTick / 1e3;
    row.latX0Us = (hiX0 - set) * nsPerTick / 1e3;
    row.spreadUs = (hi - lo) * nsPerTick / 1e3;
    row.firstUs = (lo - set) * nsPerTick / 1e3;
    row.b0Us = (r.obs[(size_t)e * blocks] - set) * nsPerTick / 1e3;
    row.e2eUs = r.uEnd[e] ? ((long long)r.uEnd[e] - set) * nsPerTick / 1e3 : -1.0;
    row.claimer = r.claim[e] - 1;
    row.site = r.site[e];
    out.push_back(row);
  }
  return out;
}

void dump_obs1(const char* path, const EventResult& r, int nEvents, int blocks,
               double wallMHz) {
  if (!path || !path[0]) return;
  FILE* f = fopen(path, "wb");
  if (!f) {
    fprintf(stderr, "warning: cannot open %s\n", path);
    return;
  }
  const double nsPerTick = 1000.0 / wallMHz;
  const long long hdr[3] = {0x3153424fLL, nEvents, blocks};
  fwrite(hdr, sizeof(long long), 3, f);
  std::vector<long long> v(nEvents);
  for (int e = 0; e < nEvents; ++e) v[e] = (long long)(r.setGT[e] * nsPerTick);
  fwrite(v.data(), sizeof(long long), nEvents, f);
  std::vector<long long> o((size_t)nEvents * blocks);
  for (size_t i = 0; i < o.size(); ++i) o[i] = r.obs[i] ? (long long)(r.obs[i] * nsPerTick) : 0;
  fwrite(o.data(), sizeof(long long), o.size(), f);
  fclose(f);
  printf("obs matrix: %s (%d events x %d blocks)\n", path, nEvents, blocks);
}

}  // namespace host
