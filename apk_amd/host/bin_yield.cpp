// yield -- preemption latency, polling overhead, exactly-once oracle and
// float64 verification of the tile-boundary yield on MI355X.
//
// Measurement surface of the reference's bin/yield (src/yield.cu:327-960):
// flags --mode latency|overhead|verify|oracle --set dev --k 64 --tiles-m 48
// --tiles-n 48 --events 10000 --tasks 200000 --reps 20 --gap-min-us 150
// --gap-max-us 400 --blocks 0 --poll-every 1|2|4|8 --warmup-events 100 --csv
// --dump-obs --urgent-tiles 1, the same stdout summary lines, the latency CSV
// "event,set_ns,first_obs_ns,last_obs_ns,lat_us,spread_us,claimer,e2e_us,
// complete,last_block,block0_delay_us,lat_excl_setter_us" (extra columns
// appended), the overhead CSV "rep,poll,wall_ms" and the OBS1 matrix.
// Additions:
//   --engine valu64|mfma128   tile engine (default valu64, the reference tile;
//                             --dtype fp32 names the same default)
//   --gemm-k K                GEMM depth walked in --k chunks (default --k)
//   --poll chunk|stage        poll at chunk boundaries (default) or every stage
//   --resume ckpt|acc|restart what a yielding block does with its tile
//   --blocks-per-cu n         workers per CU when --blocks is 0 (0 = max)
//   --arrival uniform|exp     event gaps U(gap-min,gap-max) or exponential
//   --mean-gap-us m           mean gap of the exponential arrivals
//   --urgent-m/-n/-k          urgent job shape (default tile_m x urgent-tiles*
//                             tile_n x --k: urgent-tiles tiles of depth --k)
//   --seed s                  glibc seed of A, B (21); schedule seed (21)
//   --flag-copies c           replicas of the flag (block b polls b % c)
// --set host (latency mode): the host raises each event itself (the
// reference's registered definition, src/yield.cu:837-858). The flag lives in
// host-mapped coherent memory (hipHostMalloc), the host stores the new
// generation into it and the kernel samples it at system scope. Host times
// are mapped onto the device clock with the spin_flag calibration
// (src/yield.cu:782-813): 300 times, a one-wave kernel spins on the flag, the
// host stores 1 and the kernel records the device tick at which it reads it;
// the p50 of (device time - host time) is added to every host set time.
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "host_common.hpp"
#include "yield_rig.hpp"

using namespace host;

static int poll_mode(const std::string& s) {
  if (s == "chunk" || s == "boundary" || s == "pe") return APK_POLL_CHUNK;
  if (s == "stage") return APK_POLL_STAGE;
  if (s == "off") return APK_POLL_OFF;
  return -1;
}
static int resume_mode(const std::string& s) {
  if (s == "ckpt" || s == "checkpoint") return APK_RESUME_CKPT_FULL;
  if (s == "acc") return APK_RESUME_CKPT_ACC;
  if (s == "restart") return APK_RESUME_RESTART;
  return -1;
}

int main(int argc, char** argv) {
  const std::string mode = parse_str(argc, argv, "--mode", "latency");
  const std::string setBy = parse_str(argc, argv, "--set", "dev");
  const int kChunk = (int)parse_arg(argc, argv, "--k", 64);
  const int tilesM = (int)parse_arg(argc, argv, "--tiles-m", 48);
  const int tilesN = (int)parse_arg(argc, argv, "--tiles-n", 48);
  const int events = (int)parse_arg(argc, argv, "--events", 10000);
  const unsigned tasks = (unsigned)parse_arg(argc, argv, "--tasks", 200000);
  const int reps = (int)parse_arg(argc, argv, "--reps", 20);
  const double gapMinUs = parse_arg(argc, argv, "--gap-min-us", 150);
  const double gapMaxUs = parse_arg(argc, argv, "--gap-max-us", 400);
  int blocks = (int)parse_arg(argc, argv, "--blocks", 0);
  const int pollEvery = (int)parse_arg(argc, argv, "--poll-every", 1);
  const int warmupEvents = (int)parse_arg(argc, argv, "--warmup-events", 100);
  const char* csvPath = parse_str(argc, argv, "--csv", "");
  const char* dumpObsPath = parse_str(argc, argv, "--dump-obs", "");
  const int urgentTiles = (int)parse_arg(argc, argv, "--urgent-tiles", 1);
  const std::string engName = engine_arg(argc, argv, "valu64");
  const int gemmK = (int)parse_arg(argc, argv, "--gemm-k", kChunk);
  const int poll = poll_mode(parse_str(argc, argv, "--poll", "chunk"));
  const int resume = resume_mode(parse_str(argc, argv, "--resume", "ckpt"));
  const int bpc = (int)parse_arg(argc, argv, "--blocks-per-cu", 0);
  const std::string arrival = parse_str(argc, argv, "--arrival", "uniform");
  const double meanGapUs = parse_arg(argc, argv, "--mean-gap-us", 2000);
  const unsigned seed = (unsigned)parse_arg(argc, argv, "--seed", 21);
  const int flagCopies = (int)parse_arg(argc, argv, "--flag-copies", 1);

  const int engine = engName == "mfma128" ? APK_ENGINE_MFMA128
                     : engName == "valu64" ? APK_ENGINE_VALU64 : -1;
  if (engine < 0 || poll <= 0 || resume < 0) {
    fprintf(stderr, "bad --engine, --poll or --resume\n");
    return 1;
  }
  if (setBy != "dev" && setBy != "host") {
    fprintf(stderr, "--set %s: expected dev or host\n", setBy.c_str());
    return 1;
  }
  // Host-set events exist in latency mode only (src/yield.cu:836-858); the
  // other modes use the device setter whatever --set says.
  const bool hostSet = setBy == "host" && mode == "latency";
  if (pollEvery != 1 && pollEvery != 2 && pollEvery != 4 && pollEvery != 8) {
    fprintf(stderr, "--poll-every must be 1, 2, 4, or 8\n");
    return 1;
  }
  apk_engine_geometry geo;
  APK_CHECK(apk_engine_geometry_of(engine, &geo));
  if (kChunk % geo.k_stage != 0 || gemmK % kChunk != 0) {
    fprintf(stderr, "--k must be a multiple of %d and divide --gemm-k\n", geo.k_stage);
    return 1;
  }
  const int Mu = (int)parse_arg(argc, argv, "--urgent-m", geo.tile_m);
  const int Nu = (int)parse_arg(argc, argv, "--urgent-n", urgentTiles * geo.tile_n);
  const int Ku = (int)parse_arg(argc, argv, "--urgent-k", kChunk);

  const Device dev = device_query();
  int maxPerCU = 0;
  APK_CHECK(apk_persistent_yield_occupancy(engine, poll, &maxPerCU));
  const int sat = dev.info.cu_count * maxPerCU;
  if (blocks <= 0) blocks = bpc > 0 ? dev.info.cu_count * std::min(bpc, maxPerCU) : sat;

  const int M = tilesM * geo.tile_m, N = tilesN * geo.tile_n, K = gemmK;
  const int totalTiles = tilesM * tilesN;
  if (Mu > M || Nu > N || Ku > K || Mu % geo.tile_m || Nu % geo.tile_n || Ku % geo.k_stage) {
    fprintf(stderr, "urgent job %dx%dx%d must fit the GEMM and the tile grid\n", Mu, Nu, Ku);
    return 1;
  }
  const int U = (Mu / geo.tile_m) * (Nu / geo.tile_n);
  printf("GPU: %s | %d CUs | %d blocks/CU -> sat=%d | mode=%s set=%s | K=%d k-chunk=%d "
         "blocks=%d | engine %s poll %s every %d | resume %s\n",
         dev.info.arch, dev.info.cu_count, maxPerCU, sat, mode.c_str(), setBy.c_str(), K,
         kChunk, blocks, engName.c_str(), poll == APK_POLL_STAGE ? "stage" : "chunk",
         pollEvery, parse_str(argc, argv, "--resume", "ckpt"));
  printf("urgent job: %dx%dx%d = %d tiles per event\n", Mu, Nu, Ku, U);

  std::vector<float> hA((size_t)M * K), hB((size_t)K * N);
  fill_uniform_pm1(seed, hA, hB);
  std::vector<float> hAu((size_t)Mu * Ku), hBu((size_t)Ku * Nu);
  for (int i = 0; i < Mu; ++i)
    for (int k = 0; k < Ku; ++k) hAu[(size_t)i * Ku + k] = hA[(size_t)i * K + k];
  for (int k = 0; k < Ku; ++k)
    for (int j = 0; j < Nu; ++j) hBu[(size_t)k * Nu + j] = hB[(size_t)k * N + j];

  const int evCap = std::max(events, 5);
  RigShape shape;
  shape.engine = engine;
  shape.M = M;
  shape.N = N;
  shape.K = K;
  shape.kChunk = kChunk;
  shape.Mu = Mu;
  shape.Nu = Nu;
  shape.Ku = Ku;
  shape.blocks = blocks;
  shape.events = evCap;
  shape.hashTasks = (mode == "verify") ? tasks : 0;
  shape.flagCopies = flagCopies;
  shape.hostFlag = hostSet;
  YieldRig rig(shape, hA, hB, hAu, hBu);
  hipStream_t kStream;
  HIP_CHECK(hipStreamCreateWithFlags(&kStream, hipStreamNonBlocking));
  const double flopTask = 2.0 * geo.tile_m * geo.tile_n * (double)K;

  auto timed_run = [&](int pm, unsigned nTasks, bool setter, int nEv, bool oracle,
                       long long stopTicks) {
    hipEvent_t a, b;
    HIP_CHECK(hipEventCreate(&a));
    HIP_CHECK(hipEventCreate(&b));
    const int64_t t0 = now_ns();
    HIP_CHECK(hipEventRecord(a, kStream));
    rig.launch(pm, pollEvery, resume, 0, nTasks, setter, nEv, oracle, kStream, stopTicks);
    HIP_CHECK(hipEventRecord(b, kStream));
    HIP_CHECK(hipStreamSynchronize(kStream));
    HIP_CHECK(hipGetLastError());
    float ms = 0;
    HIP_CHECK(hipEventElapsedTime(&ms, a, b));
    const double hostMs = (now_ns() - t0) / 1e6;
    HIP_CHECK(hipEventDestroy(a));
    HIP_CHECK(hipEventDestroy(b));
    return std::make_pair((double)ms, hostMs);
  };

  auto schedule = [&](int n) {
    return arrival == "exp" ? exp_schedule(21, meanGapUs, n)
                            : uniform_schedule(21, gapMinUs, gapMaxUs, n);
  };

  // float64 check of C (tiles covered) and of the urgent output.
  auto verify_outputs = [&](int coveredTiles, bool checkUrgent, double& maxRel) {
    const std::vector<float> hC = rig.readC();
    int64_t bad = 0, nans = 0;
    maxRel = 0;
    const int tN = N / geo.tile_n;
    std::vector<double> ref((size_t)geo.tile_m * N);
    for (int tr = 0; tr * tN < coveredTiles && tr < tilesM; ++tr) {
      gemm_f64(hA.data() + (size_t)tr * geo.tile_m * K, hB.data(), ref.data(), geo.tile_m,
               N, K, 0);
      const int nt = std::min(tN, coveredTiles - tr * tN);
      for (int i = 0; i < geo.tile_m; ++i)
        for (int j = 0; j < nt * geo.tile_n; ++j) {
          const float got = hC[(size_t)(tr * geo.tile_m + i) * N + j];
          const double r = ref[(size_t)i * N + j];
          if (std::isnan(got)) { ++nans; continue; }
          const double err = std::fabs(got - r);
          maxRel = std::max(maxRel, err / std::max(1.0, std::fabs(r)));
          if (err > 1e-4 + 1e-4 * std::fabs(r) && K <= 256) ++bad;
        }
    }
    int64_t ubad = 0;
    if (checkUrgent) {
      const std::vector<float> hCu = rig.readCu();
      std::vector<double> uref((size_t)Mu * Nu);
      gemm_f64(hAu.data(), hBu.data(), uref.data(), Mu, Nu, Ku, 0);
      const CheckResult cr = check(hCu.data(), uref.data(), (int64_t)uref.size(), 1e-4, 1e-4);
      ubad = cr.nans + (Ku <= 256 ? cr.bad : 0) + (cr.rel_frob > 1e-5);
      maxRel = std::max(maxRel, cr.max_rel);
    }
    return std::make_tuple(bad, nans, ubad);
  };

  // ------------------------------------------------------------ visibility
  // Notification latency with the tile work removed (src/yield.cu:468-568):
  // per event, quantiles across blocks of (observation - set), then
  // aggregated over events; plus the round trip of the polled load.
  if (mode == "visibility") {
    const int workIters = (int)parse_arg(argc, argv, "--work-iters", 0);
    const bool loadTraffic = parse_arg(argc, argv, "--loaded", 0) != 0;
    const int ldsBytes = (int)parse_arg(argc, argv, "--lds-bytes", geo.lds_bytes + 1024);
    int perCU = 0;
    APK_CHECK(apk_visibility_occupancy(ldsBytes, &perCU));
    const int vBlocks = (int)parse_arg(argc, argv, "--blocks", 0) > 0
                            ? (int)parse_arg(argc, argv, "--blocks", 0)
                            : dev.info.cu_count * perCU;
    if (vBlocks > dev.info.cu_count * perCU) {
      fprintf(stderr, "ERROR: %d blocks > %d residency slots. Refusing.\n", vBlocks,
              dev.info.cu_count * perCU);
      return 1;
    }
    const std::vector<long long> gaps = schedule(events);
    std::vector<long long> tk(events);
    for (int e = 0; e < events; ++e) tk[e] = (long long)std::llround(gaps[e] * dev.wall_mhz / 1000.0);
    const int trafficLen = 4 * 1024 * 1024;  // float4 entries: 64 MiB, DRAM-resident
    int* dFlag;
    long long *dSched, *dSet, *dObs, *dIter, *dLd;
    float *dTraffic, *dSink;
    const size_t flagBytes = (size_t)APK_FLAG_MAX_COPIES * APK_FLAG_STRIDE;
    HIP_CHECK(hipMalloc(&dFlag, flagBytes));
    HIP_CHECK(hipMalloc(&dSched, (size_t)events * 8));
    HIP_CHECK(hipMalloc(&dSet, (size_t)events * 8));
    HIP_CHECK(hipMalloc(&dObs, (size_t)events * vBlocks * 8));
    HIP_CHECK(hipMalloc(&dIter, (size_t)vBlocks * 8));
    HIP_CHECK(hipMalloc(&dLd, (size_t)vBlocks * 16));
    HIP_CHECK(hipMalloc(&dTraffic, (size_t)trafficLen * 16));
    HIP_CHECK(hipMalloc(&dSink, (size_t)vBlocks * 256 * 4));
    int* dDom;
    HIP_CHECK(hipMalloc(&dDom, (size_t)vBlocks * 4));
    {
      std::vector<float> hT((size_t)trafficLen * 4);
      for (size_t i = 0; i < (size_t)trafficLen; ++i) {
        hT[4 * i] = (float)(i % 251);
        hT[4 * i + 1] = (float)(i % 241);
        hT[4 * i + 2] = (float)(i % 239);
        hT[4 * i + 3] = (float)(i % 233);
      }
      HIP_CHECK(hipMemcpy(dTraffic, hT.data(), hT.size() * 4, hipMemcpyHostToDevice));
    }
    HIP_CHECK(hipMemcpy(dSched, tk.data(), (size_t)events * 8, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemset(dFlag, 0, flagBytes));
    HIP_CHECK(hipMemset(dSet, 0, (size_t)events * 8));
    HIP_CHECK(hipMemset(dObs, 0, (size_t)events * vBlocks * 8));
    HIP_CHECK(hipDeviceSynchronize());
    apk_vis_params vp;
    memset(&vp, 0, sizeof vp);
    vp.flag = dFlag;
    vp.flag_copies = flagCopies;
    vp.sched = dSched;
    vp.num_events = events;
    vp.stop_after = (long long)(2000.0 * dev.wall_mhz);  // 2 ms after the last event
    vp.max_ticks = tk[events - 1] + (long long)(1e6 * dev.wall_mhz);  // + 1 s
    vp.set_gt = dSet;
    vp.obs_gt = dObs;
    vp.work_iters = workIters;
    vp.loaded = loadTraffic ? 1 : 0;
    vp.traffic = dTraffic;
    vp.traffic_len = trafficLen;
    vp.sink = dSink;
    vp.iter_count = dIter;
    vp.load_ticks = dLd;
    vp.block_domain = dDom;
    const int64_t t0 = now_ns();
    APK_CHECK(apk_visibility(&vp, vBlocks, ldsBytes, kStream));
    HIP_CHECK(hipStreamSynchronize(kStream));
    HIP_CHECK(hipGetLastError());
    const double wallUs = (now_ns() - t0) / 1e3;
    std::vector<long long> hSet(events), hObs((size_t)events * vBlocks), hIt(vBlocks),
        hLd((size_t)vBlocks * 2);
    HIP_CHECK(hipMemcpy(hSet.data(), dSet, (size_t)events * 8, hipMemcpyDeviceToHost));
    HIP_CHECK(hipMemcpy(hObs.data(), dObs, hObs.size() * 8, hipMemcpyDeviceToHost));
    HIP_CHECK(hipMemcpy(hIt.data(), dIter, (size_t)vBlocks * 8, hipMemcpyDeviceToHost));
    HIP_CHECK(hipMemcpy(hLd.data(), dLd, hLd.size() * 8, hipMemcpyDeviceToHost));
    std::vector<int> hDom(vBlocks);
    HIP_CHECK(hipMemcpy(hDom.data(), dDom, (size_t)vBlocks * 4, hipMemcpyDeviceToHost));
    std::vector<double> iters(hIt.begin(), hIt.end()), ldAvg, ldMax;
    for (int b = 0; b < vBlocks; ++b) {
      ldAvg.push_back(hIt[b] ? hLd[2 * b] / (double)hIt[b] / dev.wall_mhz : 0.0);
      ldMax.push_back(hLd[2 * b + 1] / dev.wall_mhz);
    }
    printf("cadence: %.3f us/iteration (median block, %d work-iters, loaded=%d, %d blocks, "
           "%d B LDS, %d flag copies)\n", wallUs / percentile(iters, 0.5), workIters,
           loadTraffic ? 1 : 0, vBlocks, ldsBytes, flagCopies);
    printf("polled load round trip (us): block-avg p50 %.3f | p99 %.3f | max over blocks %.3f\n",
           percentile(ldAvg, 0.5), percentile(ldAvg, 0.99),
           *std::max_element(ldMax.begin(), ldMax.end()));
    std::vector<double> dmin, d50, d95, dmax;
    // Per XCD: each event's latest observation among that XCD's blocks.
    std::vector<std::vector<double>> xcdMax(APK_QUEUE_XCDS);
    int unset = 0, anomalies = 0;
    const double nsPerTick = 1000.0 / dev.wall_mhz;
    for (int e = 0; e < events; ++e) {
      if (hSet[e] == 0) { ++unset; continue; }
      std::vector<double> d;
      bool complete = true;
      for (int b = 0; b < vBlocks; ++b) {
        const long long o = hObs[(size_t)e * vBlocks + b];
        if (o == 0) { complete = false; break; }
        d.push_back((o - hSet[e]) * nsPerTick / 1e3);
      }
      if (!complete) { ++anomalies; continue; }
      if (e < warmupEvents) continue;
      std::vector<double> xm(APK_QUEUE_XCDS, -1.0);
      for (int b = 0; b < vBlocks; ++b) {
        const int x = (hDom[b] / APK_SES_PER_XCD) & (APK_QUEUE_XCDS - 1);
        xm[x] = std::max(xm[x], d[b]);
      }
      for (int x = 0; x < APK_QUEUE_XCDS; ++x)
        if (xm[x] >= 0) xcdMax[x].push_back(xm[x]);
      std::sort(d.begin(), d.end());
      dmin.push_back(d.front());
      d50.push_back(d[std::min((size_t)(0.5 * d.size()), d.size() - 1)]);
      d95.push_back(d[std::min((size_t)(0.95 * d.size()), d.size() - 1)]);
      dmax.push_back(d.back());
    }
    printf("\n--- visibility (%s): %zu events (%d unset, %d anomalies), %d blocks ---\n",
           loadTraffic ? "loaded" : "floor", dmax.size(), unset, anomalies, vBlocks);
    if (!dmax.empty())
      printf("across-block delay (us): Dmin p50 %.2f | D50 p50 %.2f | D95 p50 %.2f | Dmax p50 "
             "%.2f | Dmax p99 %.2f\n", percentile(dmin, 0.5), percentile(d50, 0.5),
             percentile(d95, 0.5), percentile(dmax, 0.5), percentile(dmax, 0.99));
    if (!dmax.empty()) {
      // The setter is block 0; the flag is an agent-scope location, so every
      // XCD's observation crosses the fabric.
      printf("per-XCD latest observation (us, p50 over events; setter on XCD %d):",
             (hDom[0] / APK_SES_PER_XCD) & (APK_QUEUE_XCDS - 1));
      for (int x = 0; x < APK_QUEUE_XCDS; ++x)
        if (!xcdMax[x].empty()) printf(" x%d %.2f", x, percentile(xcdMax[x], 0.5));
      printf("\n");
    }
    EventResult er;
    er.setGT = hSet;
    er.obs = hObs;
    dump_obs1(dumpObsPath, er, events, vBlocks, dev.wall_mhz);
    return 0;
  }

  // Probe: device time per task at this shape, to bound every run.
  rig.reset(false);
  const unsigned probeTasks = (unsigned)blocks * 8;
  const double usPerTask = timed_run(poll, probeTasks, false, 0, false, 0).first * 1e3 / probeTasks;

  // ------------------------------------------------------------ verify
  if (mode == "verify") {
    // A handful of device-set events 300 us apart (src/yield.cu:714-723),
    // compressed so that they all fire in the first half of this run.
    const int vEvents = std::min(events, 5);
    const double runUs = usPerTask * tasks;
    const long long gapNs =
        (long long)std::min(300000.0, runUs * 1e3 / (2.0 * (vEvents + 1)));
    std::vector<long long> gaps(vEvents);
    for (int e = 0; e < vEvents; ++e) gaps[e] = gapNs * (e + 1);
    printf("verify: %u tasks (~%.0f us), %d events %.1f us apart\n", tasks, runUs, vEvents,
           gapNs / 1e3);
    // Unpreempted reference run of the same kernel (poll off).
    rig.reset(true);
    timed_run(APK_POLL_OFF, tasks, false, 0, false, 0);
    const std::vector<float> cRef = rig.readC();
    const std::vector<unsigned long long> hRef = rig.readTaskHash(tasks);
    rig.reset(true);
    rig.setSchedule(gaps, dev.wall_mhz);
    timed_run(poll, tasks, true, vEvents, false, 0);
    const EventResult r = rig.readEvents(vEvents);
    int claimed = 0;
    for (int e = 0; e < vEvents; ++e) claimed += r.claim[e] != 0;
    double maxRel = 0;
    auto [bad, nans, ubad] = verify_outputs(std::min((int)tasks, totalTiles), claimed > 0, maxRel);
    const std::vector<float> cNow = rig.readC();
    const bool bitsSame = memcmp(cNow.data(), cRef.data(), cNow.size() * 4) == 0;
    const std::vector<unsigned long long> hNow = rig.readTaskHash(tasks);
    int64_t hashBad = 0;
    for (size_t t = 0; t < hNow.size(); ++t)
      if (hNow[t] != hRef[t]) ++hashBad;
    uint64_t yields = 0;
    for (int b = 0; b < blocks; ++b) yields += r.stats[(size_t)b * APK_STATS_PER_BLOCK + APK_ST_YIELDS];
    printf("yields taken: %llu | C bit-identical to the unpreempted run: %s | task "
           "fingerprints differing: %lld\n",
           (unsigned long long)yields, bitsSame ? "yes" : "NO", (long long)hashBad);
    if (nans || bad || ubad || !bitsSame || hashBad || claimed == 0) {
      fprintf(stderr, "FAIL: %lld NaN, %lld beyond tolerance, urgent bad %lld, claimed %d/%d, "
              "max rel %.3e\n", (long long)nans, (long long)bad, (long long)ubad, claimed,
              vEvents, maxRel);
      return 1;
    }
    printf("PASS: %d tiles + urgent job through the yield path (%d/%d events claimed), "
           "max rel err %.3e\n", std::min((int)tasks, totalTiles), claimed, vEvents, maxRel);
    return 0;
  }

  // ------------------------------------------------------------ overhead
  if (mode == "overhead") {
    // ABAB interleave with leader alternation; 2 warmup pairs discarded
    // (src/yield.cu:670-711). No event is ever set; wall = device time of
    // the launch (HIP events), host wall reported alongside.
    const int warmPairs = 2;
    std::vector<double> on, off, onH, offH;
    for (int r = 0; r < 2 * (reps + warmPairs); ++r) {
      const bool p = ((r / 2) % 2 == 0) ? (r % 2 == 0) : (r % 2 == 1);
      rig.reset(false);
      auto [ms, hostMs] = timed_run(p ? poll : APK_POLL_OFF, tasks, false, 0, false, 0);
      if (r >= 2 * warmPairs) {
        (p ? on : off).push_back(ms);
        (p ? onH : offH).push_back(hostMs);
      }
    }
    const double pOn = percentile(on, 0.5), pOff = percentile(off, 0.5);
    printf("drain of %u tasks, median of %d reps each (ABAB, %d warmup pairs discarded), "
           "poll-every=%d:\n", tasks, reps, warmPairs, pollEvery);
    printf("  poll ON : %.3f ms (%.2f TFLOP/s)\n  poll OFF: %.3f ms (%.2f TFLOP/s)\n", pOn,
           flopTask * tasks / (pOn * 1e-3) / 1e12, pOff,
           flopTask * tasks / (pOff * 1e-3) / 1e12);
    printf("  polling overhead: %.2f%%  (N1 cost threshold: 10%%; host wall %.2f%%)\n",
           (pOn / pOff - 1.0) * 100.0,
           (percentile(onH, 0.5) / percentile(offH, 0.5) - 1.0) * 100.0);
    if (csvPath[0]) {
      FILE* csv = fopen(csvPath, "w");
      if (csv) {
        fprintf(csv, "rep,poll,wall_ms\n");
        for (int r = 0; r < reps; ++r)
          fprintf(csv, "%d,1,%.4f\n%d,0,%.4f\n", r, on[r], r, off[r]);
        fclose(csv);
        printf("raw: %s\n", csvPath);
      }
    }
    return 0;
  }

  // ------------------------------------------------------------ oracle
  if (mode == "oracle") {
    const std::vector<long long> gaps = schedule(events);
    const double schedUs = gaps[events - 1] / 1e3;
    unsigned oTasks = (unsigned)std::min(1.5 * schedUs / usPerTask, 60e6);
    printf("oracle: probe %.3f us/task -> %u bounded tasks for a %.0f ms schedule, "
           "urgent-tiles=%d\n", usPerTask, oTasks, schedUs / 1e3, U);
    RigShape os = shape;
    os.oracleTasks = oTasks;
    YieldRig orig(os, hA, hB, hAu, hBu);
    orig.reset(true);
    orig.setSchedule(gaps, dev.wall_mhz);
    HIP_CHECK(hipDeviceSynchronize());
    orig.launch(poll, pollEvery, resume, 0, oTasks, true, events, true, kStream, 0);
    HIP_CHECK(hipStreamSynchronize(kStream));
    HIP_CHECK(hipGetLastError());
    const std::vector<int> ex = orig.readExec(oTasks);
    const std::vector<int> uex = orig.readUExec(events);
    const EventResult r = orig.readEvents(events);
    long long dup = 0, missed = 0;
    int firstBad = -1;
    for (unsigned t = 0; t < oTasks; ++t)
      if (ex[t] != 1) {
        if (ex[t] > 1) ++dup;
        else ++missed;
        if (firstBad < 0) firstBad = (int)t;
      }
    int fired = 0, badU = 0, unclaimed = 0, firstBadEv = -1;
    for (int e = 0; e < events; ++e) {
      if (r.setGT[e] == 0) continue;
      ++fired;
      if (uex[e] != U) {
        ++badU;
        if (firstBadEv < 0) firstBadEv = e;
      }
      if (r.claim[e] == 0) ++unclaimed;
    }
    printf("oracle tasks: %u checked | duplicates %lld | missed %lld", oTasks, dup, missed);
    if (firstBad >= 0) printf(" | first bad task %d (count %d)", firstBad, ex[firstBad]);
    printf("\noracle events: %d fired | urgent-count violations %d | unclaimed %d", fired,
           badU, unclaimed);
    if (firstBadEv >= 0) printf(" | first bad event %d (count %d)", firstBadEv, uex[firstBadEv]);
    printf("\n");
    const bool pass = dup == 0 && missed == 0 && badU == 0 && unclaimed == 0 && fired == events;
    printf("ORACLE: %s\n", pass ? "PASS" : "FAIL");
    return pass ? 0 : 1;
  }

  // ------------------------------------------------------------ latency
  if (mode != "latency") {
    fprintf(stderr, "unknown --mode %s\n", mode.c_str());
    return 1;
  }
  if (blocks > sat) {
    fprintf(stderr, "ERROR: %d blocks > %d residency slots; in unbounded latency mode the "
            "excess blocks never run and every event is an anomaly. Refusing.\n", blocks, sat);
    return 1;
  }
  const std::vector<long long> gaps = schedule(events);
  const double schedUs = gaps[events - 1] / 1e3;
  // Bounded even if the stop sentinel were never seen: 3x the schedule.
  const unsigned lTasks =
      (unsigned)std::min(3.0 * (schedUs + 100000.0) / usPerTask, 4.0e9);
  printf("latency: probe %.3f us/task (%.2f TFLOP/s) | schedule %.1f ms, %d events (%s) | "
         "task bound %u\n", usPerTask, flopTask / (usPerTask * 1e-6) / 1e12, schedUs / 1e3,
         events, arrival.c_str(), lTasks);
  const double nsPerTick = 1000.0 / dev.wall_mhz;
  // Host<->device clock calibration (host-set mode), on the idle GPU.
  long long offP50 = 0;
  if (hostSet) {
    long long* dOut;
    HIP_CHECK(hipMalloc(&dOut, 2 * sizeof(long long)));
    std::vector<double> offs;
    const int calReps = 300;
    const long long maxTicks = (long long)(100000.0 * dev.wall_mhz);  // 100 ms bound
    for (int rep = 0; rep < calReps; ++rep) {
      rig.hostSetFlag(0);
      APK_CHECK(apk_spin_flag(rig.dFlag(), 1, maxTicks, dOut, kStream));
      spin_for_ns(200000);  // let the spin kernel start
      const int64_t h0 = now_ns();
      rig.hostSetFlag(1);
      HIP_CHECK(hipStreamSynchronize(kStream));
      long long out[2];
      HIP_CHECK(hipMemcpy(out, dOut, sizeof out, hipMemcpyDeviceToHost));
      if (out[0] < 0) {
        fprintf(stderr, "FAIL: calibration: the device did not see the host's flag store\n");
        return 1;
      }
      offs.push_back((double)out[0] * nsPerTick - (double)h0);
    }
    const double offMin = percentile(offs, 0.0), p50 = percentile(offs, 0.5),
                 p90 = percentile(offs, 0.9);
    offP50 = (long long)p50;
    // The absolute offset is the epoch difference of the two clocks; only
    // its spread above the minimum is meaningful to read.
    printf("host->device flag visibility (%d reps, min-referenced): p50 +%.1f us | p90 "
           "+%.1f us\n", calReps, (p50 - offMin) / 1e3, (p90 - offMin) / 1e3);
    HIP_CHECK(hipFree(dOut));
  }
  rig.reset(false);
  std::vector<int64_t> hSet(events, 0);  // host-set times (host ns)
  double kernMs = 0;
  if (hostSet) {
    hipEvent_t a, b;
    HIP_CHECK(hipEventCreate(&a));
    HIP_CHECK(hipEventCreate(&b));
    HIP_CHECK(hipEventRecord(a, kStream));
    rig.launch(poll, pollEvery, resume, 0, lTasks, false, events, false, kStream, 0);
    HIP_CHECK(hipEventRecord(b, kStream));
    spin_for_ns(50LL * 1000 * 1000);  // settle into steady state
    const int64_t t0 = now_ns();
    for (int e = 0; e < events; ++e) {
      spin_until_ns(t0 + gaps[e]);
      hSet[e] = now_ns();
      rig.hostSetFlag(e + 1);
    }
    spin_for_ns(5LL * 1000 * 1000);
    rig.hostSetFlag(-1);  // stop sentinel
    HIP_CHECK(hipStreamSynchronize(kStream));
    HIP_CHECK(hipGetLastError());
    float ms = 0;
    HIP_CHECK(hipEventElapsedTime(&ms, a, b));
    kernMs = ms;
  } else {
    rig.setSchedule(gaps, dev.wall_mhz);
    const long long stopTicks = (long long)(2000.0 * dev.wall_mhz);  // 2 ms after the last event
    kernMs = timed_run(poll, lTasks, true, events, false, stopTicks).first;
  }
  EventResult r = rig.readEvents(events);
  if (hostSet)  // host clock mapped onto the device clock
    for (int e = 0; e < events; ++e)
      r.setGT[e] = (long long)std::llround(((double)hSet[e] + (double)offP50) / nsPerTick);
  dump_obs1(dumpObsPath, r, events, blocks, dev.wall_mhz);
  const std::vector<EventRow> rows = summarize_events(r, events, blocks, dev.wall_mhz);

  std::vector<double> lat, latX0, spread, e2e, firstDelay, b0Delay;
  int anomalies = 0, unset = 0, lastIsSetter = 0;
  FILE* csv = csvPath[0] ? fopen(csvPath, "w") : nullptr;
  if (csv)
    fprintf(csv, "event,set_ns,first_obs_ns,last_obs_ns,lat_us,spread_us,claimer,e2e_us,"
                 "complete,last_block,block0_delay_us,lat_excl_setter_us,claim_site\n");
  for (const EventRow& row : rows) {
    if (r.setGT[row.event] == 0) {
      ++unset;
      continue;
    }
    if (!row.complete) ++anomalies;
    if (row.complete && row.event >= warmupEvents) {
      lat.push_back(row.latUs);
      latX0.push_back(row.latX0Us);
      spread.push_back(row.spreadUs);
      firstDelay.push_back(row.firstUs);
      b0Delay.push_back(row.b0Us);
      if (row.lastBlock == 0) ++lastIsSetter;
      if (row.e2eUs >= 0) e2e.push_back(row.e2eUs);
    }
    if (csv)
      fprintf(csv, "%d,%lld,%lld,%lld,%.2f,%.2f,%d,%.2f,%d,%d,%.2f,%.2f,%d\n", row.event,
              row.setNs, row.firstNs, row.lastNs, row.latUs, row.spreadUs, row.claimer,
              row.e2eUs, row.complete, row.lastBlock, row.b0Us, row.latX0Us, row.site);
  }
  if (csv) fclose(csv);
  uint64_t yields = 0, tSave = 0, tUrg = 0, tRest = 0;
  for (int b = 0; b < blocks; ++b) {
    yields += r.stats[(size_t)b * APK_STATS_PER_BLOCK + APK_ST_YIELDS];
    tSave += r.stats[(size_t)b * APK_STATS_PER_BLOCK + APK_ST_SAVE];
    tUrg += r.stats[(size_t)b * APK_STATS_PER_BLOCK + APK_ST_URGENT];
    tRest += r.stats[(size_t)b * APK_STATS_PER_BLOCK + APK_ST_RESTORE];
  }
  printf("\n--- latency (%s-set, poll-every=%d, %d blocks): %zu events (%d warmup discarded, "
         "%d anomalies, %d unset) ---\n", setBy.c_str(), pollEvery, blocks, lat.size(),
         std::min(warmupEvents, events), anomalies, unset);
  printf("kernel %.1f ms for the %.1f ms schedule\n", kernMs, schedUs / 1e3);
  if (!lat.empty()) {
    if (!hostSet)
      printf("setter (block 0) was last observer in %.1f%% of events; its own delay p50 %.2f "
             "us\n", 100.0 * lastIsSetter / lat.size(), percentile(b0Delay, 0.5));
    printf("preemption latency set->last (us): p50 %.2f | p90 %.2f | p99 %.2f | max %.2f\n",
           percentile(lat, 0.5), percentile(lat, 0.9), percentile(lat, 0.99),
           *std::max_element(lat.begin(), lat.end()));
    if (!hostSet)
      printf("  excluding setter block 0:       p50 %.2f | p90 %.2f | p99 %.2f\n",
             percentile(latX0, 0.5), percentile(latX0, 0.9), percentile(latX0, 0.99));
    printf("first observer delay (us):        p50 %.2f | p99 %.2f\n",
           percentile(firstDelay, 0.5), percentile(firstDelay, 0.99));
    printf("observation spread first->last (us): p50 %.2f | p99 %.2f\n",
           percentile(spread, 0.5), percentile(spread, 0.99));
    if (!e2e.empty())
      printf("urgent e2e set->done (us): p50 %.2f | p99 %.2f\n", percentile(e2e, 0.5),
             percentile(e2e, 0.99));
    const double tileUs = usPerTask * blocks / (gemmK / kChunk);
    printf("tile (k-chunk) time at full residency: %.2f us -> p50 latency = %.2f tiles\n",
           tileUs, percentile(lat, 0.5) / tileUs);
  }
  if (yields)
    printf("yields: %llu | per yield: save %.2f us, urgent %.2f us, restore %.2f us\n",
           (unsigned long long)yields, tSave / dev.wall_mhz / yields,
           tUrg / dev.wall_mhz / yields, tRest / dev.wall_mhz / yields);
  if (csvPath[0]) printf("raw: %s\n", csvPath);
  return 0;
}
