// mid_common.cpp -- see mid_common.hpp. The driver behind bin/midyield
// (reference src/midyield.cu:348-793) and bin/tcyield (src/tcyield.cu:
// 384-842): modes events | verify | overhead | calibrate.
#include "mid_common.hpp"

#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>
#include <string>
#include <thread>
#include <vector>

#include "host_common.hpp"
#include "yield_rig.hpp"

namespace host {

int run_midyield(int argc, char** argv, const MidVariant& v) {
  const std::string mode = parse_str(argc, argv, "--mode", "events");
  const std::string disc = parse_str(argc, argv, "--discipline", "drain");
  const std::string pollS = parse_str(argc, argv, "--poll", "stage");
  const int kChunk = (int)parse_arg(argc, argv, "--k", v.k);
  const int tilesM = (int)parse_arg(argc, argv, "--tiles-m", v.tiles);
  const int tilesN = (int)parse_arg(argc, argv, "--tiles-n", v.tiles);
  const int events = (int)parse_arg(argc, argv, "--events", 10000);
  unsigned tasks = (unsigned)parse_arg(argc, argv, "--tasks", v.tasks);
  const int reps = (int)parse_arg(argc, argv, "--reps", 20);
  const double gapMinUs = parse_arg(argc, argv, "--gap-min-us", 150);
  const double gapMaxUs = parse_arg(argc, argv, "--gap-max-us", 400);
  int blocks = (int)parse_arg(argc, argv, "--blocks", 0);
  const int warmupEvents = (int)parse_arg(argc, argv, "--warmup-events", 100);
  const bool oracle = parse_arg(argc, argv, "--oracle", 0) != 0;
  const char* csvPath = parse_str(argc, argv, "--csv", "");
  const char* dumpObsPath = parse_str(argc, argv, "--dump-obs", "");
  const std::string engName = engine_arg(argc, argv, v.engine);
  const int gemmK = (int)parse_arg(argc, argv, "--gemm-k", kChunk);
  const std::string resumeS = parse_str(argc, argv, "--resume", "ckpt");
  const std::string arrival = parse_str(argc, argv, "--arrival", "uniform");
  const double meanGapUs = parse_arg(argc, argv, "--mean-gap-us", 2000);
  const unsigned seed = (unsigned)parse_arg(argc, argv, "--seed", 21);
  const int flagCopies = (int)parse_arg(argc, argv, "--flag-copies", 1);
  const int verifyRowsArg = (int)parse_arg(argc, argv, "--verify-rows", -1);
  // --poll boundary only: a site at every poll_every-th k-chunk boundary
  // (counted across tasks, as yield --poll-every does)
  const int pollEvery = (int)parse_arg(argc, argv, "--poll-every", 1);
  // --mode calibrate: untimed launches before the timed one (default none)
  const double prewarmMs = parse_arg(argc, argv, "--prewarm-ms", 0);
  // --fingerprints 0: no per-task fingerprint of the background (the
  // reference measures latency without one): hashing a tile in the epilogue
  // takes a block away from its poll sites for several us, which the
  // set->last latency then includes. Safety rests on the urgent outputs, the
  // float64 check of C and the oracle counts.
  const bool fingerprints = parse_arg(argc, argv, "--fingerprints", 1) != 0;

  const int engine = engName == "mfma128"    ? APK_ENGINE_MFMA128
                     : engName == "valu64"   ? APK_ENGINE_VALU64
                     : engName == "bf16x256" ? APK_ENGINE_BF16X256
                     : engName == "bf16x128" ? APK_ENGINE_BF16X128
                     : engName == "bf16x256x128" ? APK_ENGINE_BF16X256X128
                                             : -1;
  const int naive = disc == "naive" ? 1 : 0;
  const int poison = disc == "poison" ? 1 : 0;
  // off | boundary (k-chunk) | stage (after the stage wait) | issue (before
  // any wait: the window-forcing site, src/midyield.cu:246-258)
  const int poll = pollS == "off"        ? APK_POLL_OFF
                   : pollS == "boundary" ? APK_POLL_CHUNK
                   : pollS == "stage"    ? APK_POLL_STAGE
                   : pollS == "issue"    ? APK_POLL_ISSUE
                                         : -1;
  const int resume = resumeS == "ckpt" || resumeS == "checkpoint" ? APK_RESUME_CKPT_FULL
                     : resumeS == "acc"                           ? APK_RESUME_CKPT_ACC
                     : resumeS == "restart"                       ? APK_RESUME_RESTART
                                                                  : -1;
  if (pollEvery < 1) {
    fprintf(stderr, "--poll-every must be >= 1\n");
    return 1;
  }
  if (engine < 0 || poll < 0 || resume < 0 ||
      (disc != "drain" && disc != "naive" && disc != "poison")) {
    fprintf(stderr, "bad --engine, --discipline, --poll or --resume\n");
    return 1;
  }
  if (arrival != "uniform" && arrival != "exp") {
    fprintf(stderr, "unknown --arrival %s (uniform|exp)\n", arrival.c_str());
    return 1;
  }
  apk_engine_geometry geo;
  APK_CHECK(apk_engine_geometry_of(engine, &geo));
  if (kChunk % geo.k_stage != 0 || gemmK % kChunk != 0 || gemmK / geo.k_stage < 2) {
    fprintf(stderr, "--k must be a multiple of %d, divide --gemm-k, and the tile needs >= 2 "
            "k-stages\n", geo.k_stage);
    return 1;
  }
  const int Mu = (int)parse_arg(argc, argv, "--urgent-m", geo.tile_m);
  const int Nu = (int)parse_arg(argc, argv, "--urgent-n", geo.tile_n);
  const int Ku = (int)parse_arg(argc, argv, "--urgent-k", kChunk);
  if (Mu <= 0 || Nu <= 0 || Ku <= 0 || Mu % geo.tile_m || Nu % geo.tile_n || Ku % geo.k_stage) {
    fprintf(stderr, "urgent job %dx%dx%d is not a whole number of tiles\n", Mu, Nu, Ku);
    return 1;
  }
  const int U = (Mu / geo.tile_m) * (Nu / geo.tile_n);

  const Device dev = device_query();
  int maxPerCU = 0;
  APK_CHECK(apk_persistent_yield_occupancy(engine, poll == APK_POLL_OFF ? APK_POLL_STAGE : poll,
                                            &maxPerCU));
  const int sat = dev.info.cu_count * maxPerCU;
  if (blocks <= 0) blocks = sat;
  if (blocks > sat) {
    fprintf(stderr, "ERROR: %d blocks > %d residency slots\n", blocks, sat);
    return 1;
  }
  const int M = tilesM * geo.tile_m, N = tilesN * geo.tile_n, K = gemmK;
  const int totalTiles = tilesM * tilesN;
  const int S = K / geo.k_stage;
  printf("GPU: %s | %d CUs | %d blocks/CU -> sat=%d | mode=%s disc=%s poll=%s | K=%d "
         "stages=%d (k-stage %d) blocks=%d | engine %s resume %s\n",
         dev.info.arch, dev.info.cu_count, maxPerCU, sat, mode.c_str(), disc.c_str(),
         pollS.c_str(), K, S, geo.k_stage, blocks, engName.c_str(), resumeS.c_str());
  printf("urgent job per event: %dx%dx%d = %d tiles\n", Mu, Nu, Ku, U);

  // hA/hB (and hAu/hBu): the values the float64 reference multiplies, B as
  // K x N. dev*: the bytes the kernels read -- the same floats for the fp32
  // engines; bf16 bit patterns with B transposed (Bt = N x K) for the bf16 engines.
  const bool bf16 = geo.elem_bytes == 2;
  std::vector<float> hA((size_t)M * K), hB((size_t)K * N);
  std::vector<float> hAu((size_t)Mu * Ku), hBu((size_t)Ku * Nu);
  std::vector<uint8_t> devA, devB, devAu, devBu;
  if (bf16) {
    // normal(0,1) rounded to bf16 (the reference's tcyield data, src/tcyield.cu:459-473)
    std::vector<uint16_t> a, b, au, bu;
    fill_normal_bf16(seed, hA, a, hB, b);
    fill_normal_bf16(seed + 1, hAu, au, hBu, bu);
    devA = as_bytes(a);
    devB = as_bytes(transpose_u16(b, K, N));
    devAu = as_bytes(au);
    devBu = as_bytes(transpose_u16(bu, Ku, Nu));
  } else {
    fill_uniform_pm1(seed, hA, hB);
    fill_uniform_pm1(seed + 1, hAu, hBu);
    devA = as_bytes(hA);
    devB = as_bytes(hB);
    devAu = as_bytes(hAu);
    devBu = as_bytes(hBu);
  }

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
  shape.flagCopies = flagCopies;
  shape.cuPerEvent = true;
  YieldRig rig(shape, devA, devB, devAu, devBu);
  hipStream_t kStream;
  HIP_CHECK(hipStreamCreateWithFlags(&kStream, hipStreamNonBlocking));
  const int threads = (int)std::max(1u, std::thread::hardware_concurrency());

  auto timed_run = [&](int pm, unsigned nTasks, bool setter, int nEv, bool orc) {
    hipEvent_t a, b;
    HIP_CHECK(hipEventCreate(&a));
    HIP_CHECK(hipEventCreate(&b));
    HIP_CHECK(hipEventRecord(a, kStream));
    rig.launch(pm, pm == APK_POLL_CHUNK ? pollEvery : 1, resume, poison, nTasks, setter, nEv,
               orc, kStream, 0, naive);
    HIP_CHECK(hipEventRecord(b, kStream));
    HIP_CHECK(hipStreamSynchronize(kStream));
    HIP_CHECK(hipGetLastError());
    float ms = 0;
    HIP_CHECK(hipEventElapsedTime(&ms, a, b));
    HIP_CHECK(hipEventDestroy(a));
    HIP_CHECK(hipEventDestroy(b));
    return (double)ms;
  };

  // ------------------------------------------------------------ calibrate
  // Tile throughput with polling off (src/tcyield.cu:637-651).
  if (mode == "calibrate") {
    // Engine clock during the timed run: probes over 80% of its expected
    // length (apk_clock_probe). The probe stream's hardware queue is set up
    // first: set up beside a running GEMM it slows the GEMM for a while.
    ClockProbe probe;
    rig.reset(false);
    const double warmMs = timed_run(APK_POLL_OFF, (unsigned)blocks, false, 0, false);
    // --prewarm-ms: untimed launches of the timed run's size first, so that
    // the engine clock has left its idle level (it climbs over ~1 s of load).
    const int64_t preEnd = now_ns() + (int64_t)(prewarmMs * 1e6);
    int preRuns = 0;
    while (now_ns() < preEnd) {
      rig.reset(false);
      timed_run(APK_POLL_OFF, tasks, false, 0, false);
      ++preRuns;
    }
    if (preRuns) printf("pre-warm: %d untimed runs of %u tasks\n", preRuns, tasks);
    rig.reset(false);
    hipEvent_t a, b;
    HIP_CHECK(hipEventCreate(&a));
    HIP_CHECK(hipEventCreate(&b));
    HIP_CHECK(hipEventRecord(a, kStream));
    rig.launch(APK_POLL_OFF, 1, resume, 0, tasks, false, 0, false, kStream, 0, 0);
    HIP_CHECK(hipEventRecord(b, kStream));
    probe.launch(0.8 * warmMs * ((double)tasks / blocks) * 1e3, dev.wall_mhz);
    HIP_CHECK(hipDeviceSynchronize());
    HIP_CHECK(hipGetLastError());
    float fms = 0;
    HIP_CHECK(hipEventElapsedTime(&fms, a, b));
    const double ms = fms;
    const double flop = 2.0 * geo.tile_m * geo.tile_n * (double)K * tasks;
    const double peak = bf16 ? kPeakBf16TF : kPeakFp32TF;
    printf("calibrate K=%d: %u tasks on %d blocks in %.3f ms -> %.2f us/task/block | %.1f "
           "GFLOP/s (%.1f%% of %.1f TFLOP/s)\n", K, tasks, blocks, ms, ms * 1e3 * blocks / tasks,
           flop / (ms * 1e6), 100.0 * flop / (ms * 1e9) / peak, peak);
    probe.print("the run", dev.wall_mhz);
    return 0;
  }

  // ------------------------------------------------------------ overhead
  if (mode == "overhead") {
    const int warmPairs = 2;
    std::vector<double> wallOn, wallOff;
    for (int r = 0; r < 2 * (reps + warmPairs); ++r) {
      const bool on = ((r / 2) % 2 == 0) ? (r % 2 == 0) : (r % 2 == 1);
      rig.reset(false);
      const double ms = timed_run(on ? poll : APK_POLL_OFF, tasks, false, 0, false);
      if (r >= 2 * warmPairs) (on ? wallOn : wallOff).push_back(ms);
    }
    const double on = percentile(wallOn, 0.5), off = percentile(wallOff, 0.5);
    const double flop = 2.0 * geo.tile_m * geo.tile_n * (double)K * tasks;
    printf("pipelined-tile drain of %u tasks, %d reps (order-alternated):\n", tasks, reps);
    printf("  poll %s: %.3f ms | poll off: %.3f ms | overhead %.2f%%  (%.2f / %.2f TFLOP/s)\n",
           pollS.c_str(), on, off, (on / off - 1.0) * 100.0, flop / on / 1e9, flop / off / 1e9);
    if (csvPath[0]) {
      FILE* csv = fopen(csvPath, "w");
      if (csv) {
        fprintf(csv, "rep,poll,wall_ms\n");
        for (int r = 0; r < reps; ++r)
          fprintf(csv, "%d,1,%.4f\n%d,0,%.4f\n", r, wallOn[r], r, wallOff[r]);
        fclose(csv);
      }
    }
    return 0;
  }
  if (poll == APK_POLL_OFF) {
    fprintf(stderr, "--poll off is only meaningful with --mode overhead\n");
    return 1;
  }

  // --- References computed once: the urgent job on the non-preemptible
  // kernel (bitwise reference for every event's output) and in float64;
  // the background tiles' fingerprints without preemption.
  std::vector<float> uRefGpu((size_t)Mu * Nu);
  {
    void *dAu, *dBu;
    float* dCu;
    unsigned* dNx;
    HIP_CHECK(hipMalloc(&dAu, devAu.size()));
    HIP_CHECK(hipMalloc(&dBu, devBu.size()));
    HIP_CHECK(hipMalloc(&dCu, uRefGpu.size() * 4));
    HIP_CHECK(hipMalloc(&dNx, APK_QUEUE_WORDS * sizeof(unsigned)));
    HIP_CHECK(hipMemcpy(dAu, devAu.data(), devAu.size(), hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(dBu, devBu.data(), devBu.size(), hipMemcpyHostToDevice));
    HIP_CHECK(hipMemset(dNx, 0, APK_QUEUE_WORDS * sizeof(unsigned)));
    APK_CHECK(apk_persistent_gemm(engine, dAu, dBu, dCu, Mu, Nu, Ku, Ku, dNx, nullptr,
                                  std::min(U, blocks), kStream));
    HIP_CHECK(hipStreamSynchronize(kStream));
    HIP_CHECK(hipMemcpy(uRefGpu.data(), dCu, uRefGpu.size() * 4, hipMemcpyDeviceToHost));
    HIP_CHECK(hipFree(dAu));
    HIP_CHECK(hipFree(dBu));
    HIP_CHECK(hipFree(dCu));
    HIP_CHECK(hipFree(dNx));
  }
  std::vector<double> uRef((size_t)Mu * Nu);
  gemm_f64(hAu.data(), hBu.data(), uRef.data(), Mu, Nu, Ku, threads);
  const double utol = (Ku > 256 || bf16) ? 1e-3 : 1e-4;
  const double frobBar = bf16 ? 1e-2 : 1e-5;  // fp32 and bf16 bars
  // Whether one event's urgent output is corrupt, its max rel error and the
  // number of elements beyond tolerance.
  auto check_cu = [&](const std::vector<float>& cu, double& maxRel, long long& badElems) {
    const CheckResult cr = check(cu.data(), uRef.data(), (int64_t)uRef.size(), utol, utol);
    maxRel = cr.max_rel;
    badElems = cr.bad + cr.nans;
    const bool bits = memcmp(cu.data(), uRefGpu.data(), cu.size() * 4) == 0;
    return cr.nans > 0 || cr.bad > 0 || cr.rel_frob > frobBar || !bits;
  };

  rig.reserveTasks((unsigned)totalTiles, 0);
  rig.reset(true);
  timed_run(APK_POLL_OFF, (unsigned)totalTiles, false, 0, false);
  const std::vector<unsigned long long> tileHash = rig.readTaskHash((unsigned)totalTiles);
  const std::vector<float> cRef = rig.readC();

  // float64 check of C on the first `rows` rows (all rows for short K).
  const int verifyRows =
      verifyRowsArg >= 0 ? std::min(verifyRowsArg, M) : (K <= 256 ? M : std::min(M, 256));
  auto verify_C = [&](const std::vector<float>& hC) {
    std::vector<double> ref((size_t)verifyRows * N);
#pragma omp parallel for num_threads(threads) schedule(dynamic, 4)
    for (int r = 0; r < verifyRows; ++r)
      gemm_f64_rows(hA.data(), hB.data(), &ref[(size_t)r * N], N, K, r, 1);
    const double tol = (K > 256 || bf16) ? 1e-3 : 1e-4;
    const CheckResult cr = check(hC.data(), ref.data(), (int64_t)verifyRows * N, tol, tol);
    const bool ok = cr.nans == 0 && (K > 256 || cr.bad == 0) && cr.rel_frob <= frobBar;
    printf("C check (%d of %d rows vs float64): %s -- %lld NaN, %lld beyond tol, max rel "
           "%.3e, rel-Frobenius %.2e\n", verifyRows, M, ok ? "PASS" : "FAIL",
           (long long)cr.nans, (long long)cr.bad, cr.max_rel, cr.rel_frob);
    return ok;
  };
  const bool refOk = verify_C(cRef);
  if (!refOk) {
    fprintf(stderr, "FAIL: the unpreempted run does not match float64\n");
    return 1;
  }

  std::vector<long long> gaps;
  int nEv = events;
  if (mode == "verify") {
    // A handful of events 300 us apart (src/midyield.cu:573-577), compressed
    // to fit the first half of the run.
    nEv = std::min(events, 5);
    rig.reset(false);
    const unsigned probe = (unsigned)blocks * 4;
    // every block ran 4 tasks of the probe; the run takes ceil(tasks /
    // blocks) of them (not tasks * the probe's time per task, which assumes
    // far more tasks than blocks)
    const double usPerBlockTask = timed_run(poll, probe, false, 0, false) * 1e3 / 4;
    const double runUs = usPerBlockTask * ((tasks + (unsigned)blocks - 1) / (unsigned)blocks);
    const long long gapNs = (long long)std::min(300000.0, runUs * 1e3 / (2.0 * (nEv + 1)));
    for (int e = 0; e < nEv; ++e) gaps.push_back(gapNs * (e + 1));
    printf("verify: %u tasks (~%.0f us), %d events %.1f us apart\n", tasks, runUs, nEv,
           gapNs / 1e3);
  } else if (mode == "events") {
    // Size the background queue off a probe drain so the schedule fits
    // (src/midyield.cu:604-618 sizes it with 1.5x margin). The probe runs
    // twice and the second is timed: the first starts from an idle clock and
    // overstates the task time. The margin is 2x: a probe of 8 tasks per
    // block still runs slower per task than the full job does.
    rig.reset(false);
    const unsigned probe = (unsigned)blocks * 8;
    timed_run(poll, probe, false, 0, false);
    rig.reset(false);
    const double usPerTask = timed_run(poll, probe, false, 0, false) * 1e3 / probe;
    gaps = arrival == "exp" ? exp_schedule(seed, meanGapUs, nEv)
                            : uniform_schedule(seed, gapMinUs, gapMaxUs, nEv);
    const double schedUs = gaps.back() / 1e3;
    tasks = (unsigned)std::min(2.0 * schedUs / usPerTask, 4.0e9);
    printf("probe: %.3f us/task -> %u bg tasks for a %.1f ms schedule\n", usPerTask, tasks,
           schedUs / 1e3);
  } else {
    fprintf(stderr, "unknown --mode %s\n", mode.c_str());
    return 1;
  }
  const unsigned maxHashTasks = 64u << 20;
  const bool hashAll = fingerprints && tasks <= maxHashTasks;
  rig.reserveTasks(hashAll ? tasks : 0, oracle ? tasks : 0);
  if (oracle && tasks > rig.shape().oracleTasks) {
    fprintf(stderr, "oracle needs %u counters\n", tasks);
    return 1;
  }
  rig.reset(true);
  rig.setSchedule(gaps, dev.wall_mhz);
  const double runMs = timed_run(poll, tasks, true, nEv, oracle);
  const EventResult r = rig.readEvents(nEv);
  dump_obs1(dumpObsPath, r, nEv, blocks, dev.wall_mhz);  // OBS1, as yield --dump-obs
  const std::vector<EventRow> rowsE = summarize_events(r, nEv, blocks, dev.wall_mhz);

  // Background: fingerprints of every task against the unpreempted tile.
  long long hashBad = 0, hashed = 0;
  if (hashAll) {
    const std::vector<unsigned long long> h = rig.readTaskHash(tasks);
    for (unsigned t = 0; t < tasks; ++t) {
      ++hashed;
      if (h[t] != tileHash[t % (unsigned)totalTiles]) ++hashBad;
    }
  }
  const std::vector<float> cNow = rig.readC();
  const bool cBits = tasks >= (unsigned)totalTiles &&
                     memcmp(cNow.data(), cRef.data(), cNow.size() * 4) == 0;
  const bool cOk = verify_C(cNow);

  unsigned long long yields = 0, inflight = 0, stale = 0, ckpts = 0, inflightAll = 0,
                     staleAll = 0, tSave = 0, tUrg = 0, tRest = 0;
  for (int b = 0; b < blocks; ++b) {
    const unsigned long long* st = &r.stats[(size_t)b * APK_STATS_PER_BLOCK];
    yields += st[APK_ST_YIELDS];
    tSave += st[APK_ST_SAVE];
    tUrg += st[APK_ST_URGENT];
    tRest += st[APK_ST_RESTORE];
    inflight += st[APK_ST_INFLIGHT];
    stale += st[APK_ST_STALE];
    ckpts += st[APK_ST_CHECKPOINTS];
    inflightAll += st[APK_ST_INFLIGHT_ALL];
    staleAll += st[APK_ST_STALE_ALL];
  }

  std::vector<double> lat, latX0, first, e2e;
  int anomalies = 0, unset = 0, unclaimed = 0, corrupt = 0, lastIsSetter = 0;
  double worstRel = 0.0;
  FILE* csv = csvPath[0] ? fopen(csvPath, "w") : nullptr;
  if (csv) {
    if (v.tcCsv)  // src/tcyield.cu:762-763
      fprintf(csv, "event,lat_us,lat_excl_setter_us,first_us,claimer,e2e_us,bad_elems,site,"
                   "complete\n");
    else  // src/midyield.cu:699-700
      fprintf(csv, "event,lat_us,lat_excl_setter_us,first_us,claimer,e2e_us,cu_max_rel,corrupt,"
                   "complete,site\n");
  }
  for (const EventRow& row : rowsE) {
    const int e = row.event;
    if (r.setGT[e] == 0) {
      ++unset;
      continue;
    }
    if (!row.complete) ++anomalies;
    double mr = 0.0;
    long long badElems = 0;
    bool bad = false;
    if (r.claim[e]) {
      bad = check_cu(rig.readCuEvent(e), mr, badElems);
      worstRel = std::max(worstRel, mr);
      if (bad) ++corrupt;
    } else {
      ++unclaimed;
    }
    if (row.complete && e >= (mode == "verify" ? 0 : warmupEvents)) {
      lat.push_back(row.latUs);
      latX0.push_back(row.latX0Us);
      first.push_back(row.firstUs);
      if (row.lastBlock == 0) ++lastIsSetter;
      if (row.e2eUs >= 0) e2e.push_back(row.e2eUs);
    }
    if (csv && v.tcCsv)
      fprintf(csv, "%d,%.2f,%.2f,%.2f,%d,%.2f,%lld,%d,%d\n", e, row.latUs, row.latX0Us,
              row.firstUs, row.claimer, row.e2eUs, badElems + (bad && !badElems ? 1 : 0),
              row.site, row.complete);
    else if (csv)
      fprintf(csv, "%d,%.2f,%.2f,%.2f,%d,%.2f,%.3e,%d,%d,%d\n", e, row.latUs, row.latX0Us,
              row.firstUs, row.claimer, row.e2eUs, mr, bad ? 1 : 0, row.complete,
              row.site);
  }
  if (csv) fclose(csv);

  const int tested = nEv - unset - unclaimed;
  printf("\n--- %s / %s: %d events (%d unset, %d unclaimed, %d anomalies), run %.1f ms ---\n",
         disc.c_str(), pollS.c_str(), nEv, unset, unclaimed, anomalies, runMs);
  printf("SAFETY: %d/%d urgent outputs corrupt (%.2f%%) | worst rel err %.3e | bg C %s\n",
         corrupt, tested, 100.0 * corrupt / std::max(tested, 1), worstRel,
         cOk ? "PASS" : "FAIL");
  // In flight = observed: the newest stage's last direct-to-LDS load had not
  // written its LDS bytes when the drain (naive: the save) began.
  if (naive)
    printf("yields: %llu | checkpointed without a drain with a live stage still in flight: "
           "%llu | stale checkpoints resumed: %llu (of all %llu checkpoints: %llu in flight, "
           "%llu stale)\n", yields, inflight, stale, ckpts, inflightAll, staleAll);
  else
    printf("yields: %llu | a live stage was still in flight when the drain began: %llu "
           "(of all %llu checkpoints: %llu) | stale checkpoints: %llu\n", yields, inflight, ckpts,
           inflightAll, staleAll);
  if (yields)  // block averages on the device wall clock
    printf("per yield: save %.2f us, urgent %.2f us, restore %.2f us\n",
           tSave / dev.wall_mhz / yields, tUrg / dev.wall_mhz / yields,
           tRest / dev.wall_mhz / yields);
  // With tasks cycling the grid, C holds only the last pass's writes: its
  // bit-identity says nothing about the earlier passes, which the
  // fingerprints cover.
  const bool cycles = tasks > (unsigned)totalTiles;
  printf("resumed background: %lld of %lld task fingerprints differ from the unpreempted "
         "tile%s | C bit-identical to the unpreempted run: %s\n", hashBad, hashed,
         hashAll ? "" : fingerprints ? " (not hashed: too many tasks)" : " (--fingerprints 0)",
         cycles ? (cBits ? "last pass yes (tasks cycle the grid; see fingerprints)"
                         : "last pass NO (tasks cycle the grid; see fingerprints)")
                : (cBits ? "yes" : "NO"));
  if (!lat.empty()) {
    printf("latency set->last (us): p50 %.2f | p90 %.2f | p99 %.2f  (excl setter p50 %.2f, "
           "setter-last %.1f%%)\n", percentile(lat, 0.5), percentile(lat, 0.9),
           percentile(lat, 0.99), percentile(latX0, 0.5), 100.0 * lastIsSetter / lat.size());
    printf("first observer p50 %.2f us | urgent e2e p50 %.2f us\n", percentile(first, 0.5),
           e2e.empty() ? -1.0 : percentile(e2e, 0.5));
  }
  if (csvPath[0]) printf("raw: %s\n", csvPath);

  // drain: nothing may differ. poison: every urgent output must. naive is the
  // control (src/midyield.cu:741-757 reports it without failing): a resumed
  // tile may differ, but only where a checkpoint it resumed from was observed
  // stale -- so there are no more differing task fingerprints than stale
  // resumes (a task resumed stale twice differs once), and none without one.
  bool pass;
  const bool naiveExplained =
      (unsigned long long)hashBad <= stale && ((hashBad == 0) == (stale == 0));
  if (poison)
    pass = tested > 0 && corrupt == tested;
  else if (naive)
    pass = tested > 0 && corrupt == 0 && (!hashAll || naiveExplained);
  else
    pass = tested > 0 && corrupt == 0 && cOk && hashBad == 0 &&
           (cBits || tasks < (unsigned)totalTiles) && staleAll == 0;
  if (naive)
    printf("naive control: %lld corrupted tasks, %llu stale checkpoints resumed -> %s\n",
           hashBad, stale,
           naiveExplained ? "every corruption follows a stale checkpoint" : "MISMATCH");
  if (oracle) {
    const std::vector<int> ex = rig.readExec(tasks);
    const std::vector<int> ux = rig.readUExec(nEv);
    long long dup = 0, missed = 0;
    int firstBad = -1;
    for (unsigned t = 0; t < tasks; ++t)
      if (ex[t] != 1) {
        if (ex[t] > 1) ++dup;
        else ++missed;
        if (firstBad < 0) firstBad = (int)t;
      }
    int fired = 0, badU = 0;
    for (int e = 0; e < nEv; ++e) {
      if (r.setGT[e] == 0) continue;
      ++fired;
      if (ux[e] != U) ++badU;
    }
    printf("oracle tasks: %u checked | duplicates %lld | missed %lld", tasks, dup, missed);
    if (firstBad >= 0) printf(" | first bad %d (count %d)", firstBad, ex[firstBad]);
    printf("\noracle events: %d fired | urgent-count violations %d\n", fired, badU);
    const bool opass = dup == 0 && missed == 0 && badU == 0 && fired == nEv;
    printf("ORACLE: %s\n", opass ? "PASS" : "FAIL");
    pass = pass && opass;
  }
  printf("%s: %s\n", mode.c_str(), pass ? "PASS" : "FAIL");
  return pass ? 0 : 1;
}

}  // namespace host
