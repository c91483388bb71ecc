// urgent_baseline -- how long an urgent GEMM waits behind a saturating
// persistent GEMM when nothing yields (the no-preemption baseline).
//
// Measurement surface of the reference's bin/urgent_baseline
// (src/urgent_baseline.cu:144-378): flags --k 64 --tiles-m 48 --tiles-n 48
// --bg-tasks 20000 --trials 500 --mode sat|sat-1|1persm --blocks 0
// --reserve -1 --urgent-blocks 1 --csv, the same stdout summary lines and
// the CSV "trial,delay_us,consumed_at_arrival,remaining_at_arrival,e2e_us,
// exec_us,gap_us,drain_us". Per trial the background persistent GEMM is
// launched on one stream; after a delay (uniform in 0.2..0.8 of the measured
// drain, mt19937(seed)) the urgent job is submitted on a second stream, and
// the host times arrival -> completion (e2e). Device timeline: gap = urgent
// start - background exit, exec = urgent duration, drain = background run.
//
// MI355X differences:
//  * both streams have the default priority (stream priorities are not used
//    on this pool); the urgent kernel is still only dispatched once CUs free
//    up, which is exactly what this baseline measures;
//  * the background is the preemptible kernel with polling off (tasks cycle
//    the tile grid, src/urgent_baseline.cu:78-80), the urgent job is
//    apk_persistent_gemm with --urgent-blocks workers over its own tiles.
// Additions: --engine valu64|mfma128|bf16x256|bf16x128|bf16x256x128 (or --dtype fp32|bf16),
// --gemm-k K (background depth, walked
// in --k chunks), --urgent-m/-n/-k (urgent GEMM shape; default
// urgent-blocks tiles of depth --gemm-k, as the reference), --arrival
// uniform|exp with --mean-gap-us (exponential delays, redrawn until they fall
// inside the drain), --seed, --verify-rows.
//
// --yield 1 is the same experiment with preemption on (the retreat arm): the
// background polls the flag (--poll stage|chunk, --poll-every), and the
// urgent stream carries [raise flag -> urgent GEMM -> continuation]. At the
// flag, ceil(R / 32) blocks in each of the 32 (XCD, shader engine) dispatch
// domains (R = --retreat, default --urgent-blocks: the urgent kernel's
// workgroups land in R domains that cannot be named in advance) checkpoint
// their tile (--resume
// ckpt|acc|restart) into the HBM resume queue and exit, the urgent GEMM is
// dispatched onto their CUs, and the continuation relaunches as many workers,
// which join the job; resumed tiles are finished by whichever worker pops
// them. Per trial it checks every task's fingerprint against an
// unpreempted run and (--oracle 1) that every task completed exactly once.
// CSV columns appended: raise_to_ustart_us (flag raised -> first urgent tile
// starts, device clock), retreat_first_us, retreat_last_us (flag -> first /
// last retreating block's checkpoint start / exit), retreats,
// urgent_block_xcd (per urgent tile: the urgent block that ran it and its XCD),
// retreat_xcds (the domain xcd*4+se of each retreating block), urgent_end_us, cont_start_us
// (flag -> last urgent tile done, flag -> continuation's block 0 starts).
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "host_common.hpp"
#include "yield_rig.hpp"

using namespace host;

int main(int argc, char** argv) {
  const int kChunk = (int)parse_arg(argc, argv, "--k", 64);
  const int tilesM = (int)parse_arg(argc, argv, "--tiles-m", 48);
  const int tilesN = (int)parse_arg(argc, argv, "--tiles-n", 48);
  const int bgTasks = (int)parse_arg(argc, argv, "--bg-tasks", 20000);
  const int trials = (int)parse_arg(argc, argv, "--trials", 500);
  const std::string mode = parse_str(argc, argv, "--mode", "sat");
  int blocks = (int)parse_arg(argc, argv, "--blocks", 0);
  const int reserve = (int)parse_arg(argc, argv, "--reserve", -1);
  const int urgentBlocks = (int)parse_arg(argc, argv, "--urgent-blocks", 1);
  const char* csvPath = parse_str(argc, argv, "--csv", "");
  const std::string engName = engine_arg(argc, argv, "valu64");
  const int gemmK = (int)parse_arg(argc, argv, "--gemm-k", kChunk);
  const std::string arrival = parse_str(argc, argv, "--arrival", "uniform");
  const double meanGapUs = parse_arg(argc, argv, "--mean-gap-us", 2000);
  const unsigned seed = (unsigned)parse_arg(argc, argv, "--seed", 21);
  const int verifyRows = (int)parse_arg(argc, argv, "--verify-rows", 0);
  const bool yieldArm = parse_arg(argc, argv, "--yield", 0) != 0;
  const std::string pollS = parse_str(argc, argv, "--poll", "stage");
  const int pollEvery = (int)parse_arg(argc, argv, "--poll-every", 1);
  const std::string resumeS = parse_str(argc, argv, "--resume", "ckpt");
  const int retreatN = (int)parse_arg(argc, argv, "--retreat", urgentBlocks);
  const bool oracle = parse_arg(argc, argv, "--oracle", 0) != 0;
  // --continuous 1 (with --yield 1): one background job, --events arrivals
  const bool continuous = parse_arg(argc, argv, "--continuous", 0) != 0;
  const int events = (int)parse_arg(argc, argv, "--events", 10000);
  const int poll = pollS == "stage" ? APK_POLL_STAGE : pollS == "chunk" ? APK_POLL_CHUNK : -1;
  const int resume = resumeS == "ckpt"      ? APK_RESUME_CKPT_FULL
                     : resumeS == "acc"     ? APK_RESUME_CKPT_ACC
                     : resumeS == "restart" ? APK_RESUME_RESTART
                                            : -1;
  if (yieldArm && (poll < 0 || resume < 0 || retreatN < 1 || pollEvery < 1)) {
    fprintf(stderr, "bad --poll (stage|chunk), --resume (ckpt|acc|restart), --retreat or "
            "--poll-every\n");
    return 1;
  }

  const int engine = engName == "mfma128"    ? APK_ENGINE_MFMA128
                     : engName == "valu64"   ? APK_ENGINE_VALU64
                     : engName == "bf16x256" ? APK_ENGINE_BF16X256
                     : engName == "bf16x128" ? APK_ENGINE_BF16X128
                     : engName == "bf16x256x128" ? APK_ENGINE_BF16X256X128
                                             : -1;
  if (engine < 0) {
    fprintf(stderr, "unknown --engine %s (valu64|mfma128|bf16x256|bf16x128|bf16x256x128)\n",
            engName.c_str());
    return 1;
  }
  apk_engine_geometry geo;
  APK_CHECK(apk_engine_geometry_of(engine, &geo));
  if (kChunk <= 0 || kChunk % geo.k_stage != 0 || gemmK % kChunk != 0) {
    fprintf(stderr, "--k must be a multiple of %d and divide --gemm-k\n", geo.k_stage);
    return 1;
  }
  if (arrival != "uniform" && arrival != "exp") {
    fprintf(stderr, "unknown --arrival %s (uniform|exp)\n", arrival.c_str());
    return 1;
  }
  const int urgentM = (int)parse_arg(argc, argv, "--urgent-m", geo.tile_m);
  const int urgentN = (int)parse_arg(argc, argv, "--urgent-n", urgentBlocks * geo.tile_n);
  const int urgentK = (int)parse_arg(argc, argv, "--urgent-k", gemmK);
  if (urgentM % geo.tile_m || urgentN % geo.tile_n || urgentK % geo.k_stage || urgentM <= 0 ||
      urgentN <= 0 || urgentK <= 0) {
    fprintf(stderr, "urgent job %dx%dx%d is not a whole number of %dx%dx%d tiles\n", urgentM,
            urgentN, urgentK, geo.tile_m, geo.tile_n, geo.k_stage);
    return 1;
  }
  const int uTiles = (urgentM / geo.tile_m) * (urgentN / geo.tile_n);

  const Device dev = device_query();
  int maxPerCU = 0;
  APK_CHECK(apk_persistent_yield_occupancy(engine, yieldArm ? poll : APK_POLL_OFF, &maxPerCU));
  const int sat = dev.info.cu_count * maxPerCU;
  if (blocks <= 0) {
    if (reserve >= 0) blocks = sat - reserve;
    else if (mode == "sat") blocks = sat;
    else if (mode == "sat-1") blocks = sat - 1;
    else if (mode == "1persm") blocks = dev.info.cu_count;
    else {
      fprintf(stderr, "unknown --mode %s\n", mode.c_str());
      return 1;
    }
  }
  if (blocks <= 0 || blocks > sat) {
    fprintf(stderr, "ERROR: %d blocks outside 1..%d residency slots\n", blocks, sat);
    return 1;
  }

  const int M = tilesM * geo.tile_m, N = tilesN * geo.tile_n, K = gemmK;
  printf("GPU: %s | %d CUs | %d resident blocks/CU max -> %d slots\n", dev.info.arch,
         dev.info.cu_count, maxPerCU, sat);
  printf("mode=%s: %d blocks | reserve=%d urgent-blocks=%d | K=%d (k-chunk %d) | "
         "bg-tasks=%d | trials=%d | engine %s | urgent %dx%dx%d (%d tiles)\n",
         mode.c_str(), blocks, reserve, urgentBlocks, K, kChunk, bgTasks, trials,
         engName.c_str(), urgentM, urgentN, urgentK, uTiles);
  printf("stream priorities: none (both streams at the default priority)\n");

  // hA/hB (hAu/hBu): the values the float64 reference multiplies, B as
  // K x N. dev*: the bytes the kernels read -- the same floats for the fp32
  // engines; bf16 bit patterns with B transposed (Bt = N x K) for the bf16 engines.
  const bool bf16 = geo.elem_bytes == 2;
  std::vector<float> hA((size_t)M * K), hB((size_t)K * N);
  std::vector<float> hAu((size_t)urgentM * urgentK), hBu((size_t)urgentK * urgentN);
  std::vector<uint8_t> devA, devB, devAu, devBu;
  if (bf16) {
    // normal(0,1) rounded to bf16 (the reference's tcyield data, src/tcyield.cu:459-473)
    std::vector<uint16_t> a, b, au, bu;
    fill_normal_bf16(seed, hA, a, hB, b);
    fill_normal_bf16(seed + 1, hAu, au, hBu, bu);
    devA = as_bytes(a);
    devB = as_bytes(transpose_u16(b, K, N));
    devAu = as_bytes(au);
    devBu = as_bytes(transpose_u16(bu, urgentK, urgentN));
  } else {
    fill_uniform_pm1(seed, hA, hB);
    fill_uniform_pm1(seed + 1, hAu, hBu);
    devA = as_bytes(hA);
    devB = as_bytes(hB);
    devAu = as_bytes(hAu);
    devBu = as_bytes(hBu);
  }

  RigShape rs;
  rs.engine = engine;
  rs.M = M;
  rs.N = N;
  rs.K = K;
  rs.kChunk = kChunk;
  rs.blocks = blocks;
  rs.events = (yieldArm && continuous) ? std::max(events, 1) : 1;
  rs.runTimes = true;
  // Blocks that retreat per event: ceil(R / 32) in each of the 32 (XCD,
  // shader engine) dispatch domains.
  const int retreatBlocks =
      APK_RETREAT_DOMAINS * ((retreatN + APK_RETREAT_DOMAINS - 1) / APK_RETREAT_DOMAINS);
  if (yieldArm) {
    // one event's retreats per trial; a continuous job keeps four events'
    // worth of entries in its ring (each event's are read back well before
    // the next arrival)
    rs.retreatCap = (unsigned)(continuous ? 4 * retreatBlocks : retreatBlocks);
    if (continuous && resume == APK_RESUME_RESTART) {
      // no checkpoints to hold: an entry per retreat of the whole job, so
      // that no ticket waits for its entry to come free
      rs.retreatCap = (unsigned)retreatBlocks * (unsigned)(std::max(events, 1) + 8);
      rs.retreatSlots = false;
    }
    rs.extraRows = retreatBlocks + blocks;  // continuation + drain relaunch
    rs.hashTasks = (unsigned)bgTasks;
    if (oracle) rs.oracleTasks = (unsigned)bgTasks;
  }
  YieldRig rig(rs, devA, devB, {}, {});

  void *dAu, *dBu;
  float* dCu;
  unsigned* dUNext;
  apk_tile_record* dULog;
  const int uChunks = 1;
  HIP_CHECK(hipMalloc(&dAu, devAu.size()));
  HIP_CHECK(hipMalloc(&dBu, devBu.size()));
  HIP_CHECK(hipMalloc(&dCu, (size_t)urgentM * urgentN * 4));
  HIP_CHECK(hipMalloc(&dUNext, APK_QUEUE_WORDS * sizeof(unsigned)));
  HIP_CHECK(hipMalloc(&dULog, (size_t)uTiles * uChunks * sizeof(apk_tile_record)));
  HIP_CHECK(hipMemcpy(dAu, devAu.data(), devAu.size(), hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(dBu, devBu.data(), devBu.size(), hipMemcpyHostToDevice));
  unsigned* hConsumed;  // pinned, for the mid-flight queue snapshot (per-XCD counters)
  HIP_CHECK(hipHostMalloc((void**)&hConsumed, APK_QUEUE_WORDS * sizeof(unsigned),
                          hipHostMallocDefault));

  hipStream_t bgStream, uStream;
  HIP_CHECK(hipStreamCreateWithFlags(&bgStream, hipStreamNonBlocking));
  HIP_CHECK(hipStreamCreateWithFlags(&uStream, hipStreamNonBlocking));

  auto launch_bg = [&]() {
    if (yieldArm)
      rig.launchRetreat(poll, pollEvery, resume, (unsigned)bgTasks, retreatN, 1, oracle, blocks,
                        0, false, rig.dRunGT(), rig.dExitCount(), bgStream);
    else
      rig.launch(APK_POLL_OFF, 1, APK_RESUME_RESTART, 0, (unsigned)bgTasks, false, 0, false,
                 bgStream);
  };
  auto launch_urgent = [&]() {
    HIP_CHECK(hipMemsetAsync(dUNext, 0, APK_QUEUE_WORDS * sizeof(unsigned), uStream));
    APK_CHECK(apk_persistent_gemm(engine, dAu, dBu, dCu, urgentM, urgentN, urgentK, urgentK,
                                  dUNext, dULog, urgentBlocks, uStream));
  };
  // Urgent job timeline from its per-tile records: earliest start, latest end.
  auto urgent_window = [&]() {
    std::vector<apk_tile_record> rec((size_t)uTiles * uChunks);
    HIP_CHECK(hipMemcpy(rec.data(), dULog, rec.size() * sizeof(apk_tile_record),
                        hipMemcpyDeviceToHost));
    long long s = rec[0].start, e = rec[0].end;
    for (const auto& r : rec) {
      s = std::min<long long>(s, r.start);
      e = std::max<long long>(e, r.end);
    }
    return std::make_pair(s, e);
  };
  // Which XCD each urgent tile ran on and which urgent block ran it, as
  // "block:xcd" pairs in tile order (hw slot bits [9:6] hold the XCC id).
  auto urgent_placement = [&]() {
    std::vector<apk_tile_record> rec((size_t)uTiles * uChunks);
    HIP_CHECK(hipMemcpy(rec.data(), dULog, rec.size() * sizeof(apk_tile_record),
                        hipMemcpyDeviceToHost));
    std::string out;
    for (const auto& r : rec) {
      if (!out.empty()) out += ' ';
      out += std::to_string(r.block) + ":" + std::to_string((r.smid >> 6) & 15);
    }
    return out;
  };
  const double tickUs = 1.0 / dev.wall_mhz;

  // --- Correctness gate (once, before any timing): both kernels vs float64.
  {
    printf("verifying bg + urgent kernels against float64 host reference...\n");
    rig.reset(true);
    HIP_CHECK(hipMemset(dCu, 0xFF, (size_t)urgentM * urgentN * 4));
    HIP_CHECK(hipDeviceSynchronize());
    launch_bg();
    launch_urgent();
    HIP_CHECK(hipDeviceSynchronize());
    const std::vector<float> hC = rig.readC();
    std::vector<float> hCu((size_t)urgentM * urgentN);
    HIP_CHECK(hipMemcpy(hCu.data(), dCu, hCu.size() * 4, hipMemcpyDeviceToHost));
    const int covered = std::min(bgTasks, tilesM * tilesN);
    const int coveredRows = (covered / tilesN) * geo.tile_m;
    const int rows = verifyRows > 0 ? std::min(verifyRows, coveredRows) : coveredRows;
    const int threads = (int)std::max(1u, std::thread::hardware_concurrency());
    std::vector<double> ref((size_t)rows * N);
#pragma omp parallel for num_threads(threads) schedule(dynamic, 8)
    for (int r = 0; r < rows; ++r) gemm_f64_rows(hA.data(), hB.data(), &ref[(size_t)r * N], N, K, r, 1);
    std::vector<double> uref((size_t)urgentM * urgentN);
    gemm_f64(hAu.data(), hBu.data(), uref.data(), urgentM, urgentN, urgentK, threads);
    // Elementwise gate; rel-Frobenius is the bar (fp32 1e-5, bf16 1e-2 on the
    // bf16-rounded inputs, which the float64 reference multiplies exactly).
    const double tol = (K > 256 || bf16) ? 1e-3 : 1e-4;
    const double bar = bf16 ? 1e-2 : 1e-5;
    const CheckResult cb = check(hC.data(), ref.data(), (int64_t)rows * N, tol, tol);
    const CheckResult cu = check(hCu.data(), uref.data(), (int64_t)uref.size(), tol, tol);
    if (cb.nans || cb.bad || cu.nans || cu.bad || cb.rel_frob > bar || cu.rel_frob > bar) {
      fprintf(stderr, "FAIL: bg %lld NaN %lld bad (rel-Frob %.2e); urgent %lld NaN %lld bad "
              "(rel-Frob %.2e)\n", (long long)cb.nans, (long long)cb.bad, cb.rel_frob,
              (long long)cu.nans, (long long)cu.bad, cu.rel_frob);
      return 1;
    }
    printf("PASS: %d bg rows + %d urgent tiles, max rel err %.3e / %.3e, rel-Frobenius "
           "%.2e / %.2e\n", rows, uTiles, cb.max_rel, cu.max_rel, cb.rel_frob, cu.rel_frob);
  }

  // --- Drain estimate (bg alone, device timeline), used to place arrivals.
  rig.reset(false);
  launch_bg();
  HIP_CHECK(hipStreamSynchronize(bgStream));
  auto [bs0, be0] = rig.readRunGT();
  const double drainEstUs = (be0 - bs0) * tickUs;
  printf("bg drain, no urgent: %.0f us for %d tasks on %d blocks\n", drainEstUs, bgTasks,
         blocks);

  if (yieldArm && continuous) {
    // --- Retreat arm, continuous: one background job on all workers, and the
    // host raises each of `events` arrivals (exponential gaps, --mean-gap-us)
    // as it falls due: [raise flag -> urgent GEMM] on the urgent stream, then
    // the continuation that brings the retreated workers back on a third
    // stream ordered after the urgent GEMM. The urgent GEMM is the reference's
    // urgent_tile (apk_urgent_gemm: one block per tile, no queue to clear),
    // whose start is stamped at block 0's first instruction as the
    // reference stamps it (src/urgent_baseline.cu:104).
    const int T = tilesM * tilesN;
    const std::vector<unsigned long long> tileHash = [&] {
      rig.reserveTasks((unsigned)T, 0);
      rig.reset(false);
      rig.launchRetreat(poll, pollEvery, resume, (unsigned)T, retreatN, events, false, blocks, 0,
                        false, rig.dRunGT(), rig.dExitCount(), bgStream);
      HIP_CHECK(hipStreamSynchronize(bgStream));
      return rig.readTaskHash((unsigned)T);
    }();
    std::vector<float> uRefBits((size_t)urgentM * urgentN);
    {
      HIP_CHECK(hipMemsetAsync(dUNext, 0, APK_QUEUE_WORDS * sizeof(unsigned), uStream));
      APK_CHECK(apk_persistent_gemm(engine, dAu, dBu, dCu, urgentM, urgentN, urgentK, urgentK,
                                    dUNext, nullptr, urgentBlocks, uStream));
      HIP_CHECK(hipStreamSynchronize(uStream));
      HIP_CHECK(hipMemcpy(uRefBits.data(), dCu, uRefBits.size() * 4, hipMemcpyDeviceToHost));
    }
    const std::vector<long long> gaps = arrival == "exp"
                                            ? exp_schedule(seed, meanGapUs, events)
                                            : uniform_schedule(seed, 150, 400, events);
    const double settleUs = 20000.0, schedUs = gaps.back() / 1e3;
    const double usPerTask = drainEstUs / bgTasks;
    // Sized to outlast the schedule with margin (the drain estimate, taken on
    // a cold clock over a short drain, overstates the task time by up to a
    // third); arrivals that still find the job finished are reported and left
    // out of the latency.
    const unsigned jobTasks =
        (unsigned)std::min(1.6 * (settleUs + schedUs + 20000.0) / usPerTask, 2.0e9);
    rig.reserveTasks(jobTasks, oracle ? jobTasks : 0);
    const int keepCu = std::min(events, 64);  // urgent outputs kept per event
    float* dCuAll;
    long long* dRunC;
    unsigned* dExitC;
    long long* dUStartAll;           // per arrival: urgent block 0's first instruction
    unsigned long long* dUEndAll;    // per arrival: the last urgent tile stored
    HIP_CHECK(hipMalloc(&dCuAll, (size_t)(keepCu + 1) * urgentM * urgentN * 4));
    HIP_CHECK(hipMalloc(&dRunC, 2 * (size_t)events * sizeof(long long)));
    HIP_CHECK(hipMalloc(&dExitC, (size_t)events * sizeof(unsigned)));
    HIP_CHECK(hipMalloc(&dUStartAll, (size_t)events * sizeof(long long)));
    HIP_CHECK(hipMalloc(&dUEndAll, (size_t)events * sizeof(unsigned long long)));
    HIP_CHECK(hipMemset(dCuAll, 0xFF, (size_t)(keepCu + 1) * urgentM * urgentN * 4));
    HIP_CHECK(hipMemset(dRunC, 0, 2 * (size_t)events * sizeof(long long)));
    HIP_CHECK(hipMemset(dExitC, 0, (size_t)events * sizeof(unsigned)));
    HIP_CHECK(hipMemset(dUStartAll, 0, (size_t)events * sizeof(long long)));
    HIP_CHECK(hipMemset(dUEndAll, 0, (size_t)events * sizeof(unsigned long long)));
    hipStream_t cStream;
    HIP_CHECK(hipStreamCreateWithFlags(&cStream, hipStreamNonBlocking));
    hipEvent_t evU;
    HIP_CHECK(hipEventCreateWithFlags(&evU, hipEventDisableTiming));
    printf("continuous retreat arm: %d arrivals (%s, mean %.0f us) over one job of %u tasks "
           "(%.0f us/task aggregate), %d retreats per arrival, resume ring of %u entries\n",
           events, arrival.c_str(), meanGapUs, jobTasks, usPerTask, retreatBlocks,
           rig.shape().retreatCap);

    rig.reset(false);
    rig.launchRetreat(poll, pollEvery, resume, jobTasks, retreatN, events, oracle, blocks, 0,
                      false, rig.dRunGT(), rig.dExitCount(), bgStream);
    spin_for_ns((int64_t)(settleUs * 1e3));
    const int64_t t0 = now_ns();
    for (int e = 0; e < events; ++e) {
      spin_until_ns(t0 + gaps[e]);
      float* cu = dCuAll + (size_t)std::min(e, keepCu) * urgentM * urgentN;
      APK_CHECK(apk_raise_flag(rig.dFlag(), 1, e + 1, rig.dSetGT() + e, uStream));
      // the reference's urgent_tile: one block per tile, start stamped at
      // block 0's first instruction (src/urgent_baseline.cu:100-112)
      APK_CHECK(apk_urgent_gemm(engine, dAu, dBu, cu, urgentM, urgentN, urgentK,
                                dUStartAll + e, dUEndAll + e, uStream));
      HIP_CHECK(hipEventRecord(evU, uStream));
      HIP_CHECK(hipStreamWaitEvent(cStream, evU, 0));
      rig.launchRetreat(poll, pollEvery, resume, jobTasks, retreatN, events, oracle,
                        retreatBlocks, blocks, true, dRunC + 2 * (size_t)e, dExitC + e, cStream,
                        e + 1);
    }
    HIP_CHECK(hipStreamSynchronize(uStream));
    HIP_CHECK(hipStreamSynchronize(cStream));
    HIP_CHECK(hipStreamSynchronize(bgStream));
    RetreatResult rr = rig.readRetreat(events);
    int lateDrains = 0;
    while (rr.tail > rr.head && lateDrains < 4) {
      // a block retreated after every worker had left: finish its tile
      ++lateDrains;
      rig.launchRetreat(poll, pollEvery, resume, jobTasks, retreatN, events, oracle, blocks,
                        blocks, true, nullptr, nullptr, bgStream, events);
      HIP_CHECK(hipStreamSynchronize(bgStream));
      rr = rig.readRetreat(events);
    }
    HIP_CHECK(hipGetLastError());

    auto [jobStart, bgEnd] = rig.readRunGT();
    std::vector<long long> runC(2 * (size_t)events);
    HIP_CHECK(hipMemcpy(runC.data(), dRunC, runC.size() * 8, hipMemcpyDeviceToHost));
    long long jobEnd = bgEnd;
    for (int e = 0; e < events; ++e) jobEnd = std::max(jobEnd, runC[2 * (size_t)e + 1]);
    std::vector<long long> uStart(events);
    std::vector<unsigned long long> uEnd(events);
    HIP_CHECK(hipMemcpy(uStart.data(), dUStartAll, events * sizeof(long long),
                        hipMemcpyDeviceToHost));
    HIP_CHECK(hipMemcpy(uEnd.data(), dUEndAll, events * sizeof(unsigned long long),
                        hipMemcpyDeviceToHost));
    std::vector<double> raise, uend, rfirst, rlast, cont;
    int afterJob = 0, noRetreat = 0, notRun = 0;
    FILE* csv = csvPath[0] ? fopen(csvPath, "w") : nullptr;
    if (csv)
      fprintf(csv, "event,set_ns,raise_to_ustart_us,urgent_end_us,retreat_first_us,"
                   "retreat_last_us,retreats,cont_start_us,in_job\n");
    for (int e = 0; e < events; ++e) {
      const long long set = rr.setGT[e];
      const long long us = uStart[e], ue = (long long)uEnd[e];
      if (set == 0 || ue == 0) {
        ++notRun;
        continue;
      }
      int nr = 0;
      for (int d = 0; d < APK_RETREAT_DOMAINS; ++d)
        nr += std::min(rr.count[(size_t)e * APK_RETREAT_DOMAINS + d],
                       retreatBlocks / APK_RETREAT_DOMAINS);
      const bool inJob = set < jobEnd;
      const double rf = nr ? (rr.retreatGT[2 * (size_t)e] - set) * tickUs : -1.0;
      const double rl = nr ? (rr.retreatGT[2 * (size_t)e + 1] - set) * tickUs : -1.0;
      const double cs = runC[2 * (size_t)e] ? (runC[2 * (size_t)e] - set) * tickUs : -1.0;
      if (!inJob) {
        ++afterJob;
      } else {
        if (nr == 0) ++noRetreat;
        raise.push_back((us - set) * tickUs);
        uend.push_back((ue - set) * tickUs);
        if (nr) {
          rfirst.push_back(rf);
          rlast.push_back(rl);
        }
        if (cs >= 0) cont.push_back(cs);
      }
      if (csv)
        fprintf(csv, "%d,%lld,%.2f,%.2f,%.2f,%.2f,%d,%.2f,%d\n", e,
                (long long)(set * tickUs * 1e3), (us - set) * tickUs, (ue - set) * tickUs, rf,
                rl, nr, cs, inJob ? 1 : 0);
    }
    if (csv) fclose(csv);

    // Safety: every task's fingerprint against its tile's unpreempted one,
    // every task exactly once, the kept urgent outputs bit for bit.
    const std::vector<unsigned long long> h = rig.readTaskHash(jobTasks);
    long long hashBad = 0, oracleBad = 0, uBad = 0;
    for (unsigned i = 0; i < jobTasks; ++i) hashBad += h[i] != tileHash[i % (unsigned)T];
    if (oracle) {
      const std::vector<int> ex = rig.readExec(jobTasks);
      for (unsigned i = 0; i < jobTasks; ++i) oracleBad += ex[i] != 1;
    }
    {
      std::vector<float> cu((size_t)(keepCu + 1) * urgentM * urgentN);
      HIP_CHECK(hipMemcpy(cu.data(), dCuAll, cu.size() * 4, hipMemcpyDeviceToHost));
      const size_t n = (size_t)urgentM * urgentN;
      for (int k = 0; k <= keepCu; ++k)
        if (k < events) uBad += memcmp(cu.data() + k * n, uRefBits.data(), n * 4) != 0;
    }
    const EventResult er = rig.readEvents(0);
    unsigned long long retreats = 0, resumed = 0, errors = 0, saveTicks = 0, declined = 0;
    for (int b = 0; b < blocks + rs.extraRows; ++b) {
      const unsigned long long* st = &er.stats[(size_t)b * APK_STATS_PER_BLOCK];
      retreats += st[APK_ST_RETREATS];
      resumed += st[APK_ST_RESUMED];
      errors += st[APK_ST_ERRORS];
      declined += st[APK_ST_DECLINED];
      saveTicks += st[APK_ST_SAVE];
    }
    // The background alone again, now that the engine clock has settled
    // under the job (the drain estimate before it started from a cold clock
    // and overstates the task time): the reference for the overhead and the
    // tile time.
    // A sixteenth of the job (over a second of work), so that the launch and
    // the drain's tail (the last tasks run on fewer workers) weigh as little
    // as they do in the job.
    const unsigned aloneTasks = std::min(jobTasks, std::max((unsigned)bgTasks, jobTasks / 16));
    rig.reset(false);
    rig.resetRetreat();
    rig.launchRetreat(poll, pollEvery, resume, aloneTasks, retreatN, 1, false, blocks, 0, false,
                      rig.dRunGT(), rig.dExitCount(), bgStream);
    HIP_CHECK(hipStreamSynchronize(bgStream));
    HIP_CHECK(hipGetLastError());
    const auto [as0, ae0] = rig.readRunGT();
    const double usPerTaskWarm = (ae0 - as0) * tickUs / aloneTasks;
    // The same length on the kernel with polls off, against which every
    // arm's cost is stated.
    rig.reset(false);
    rig.launch(APK_POLL_OFF, 1, APK_RESUME_RESTART, 0, aloneTasks, false, 0, false, bgStream);
    HIP_CHECK(hipStreamSynchronize(bgStream));
    HIP_CHECK(hipGetLastError());
    const auto [os0, oe0] = rig.readRunGT();
    const double usPerTaskOff = (oe0 - os0) * tickUs / aloneTasks;
    const double jobUs = (jobEnd - jobStart) * tickUs;
    const double flopTask = 2.0 * geo.tile_m * geo.tile_n * (double)K;
    const double tfJob = flopTask * jobTasks / (jobUs * 1e-6) / 1e12;
    const double tfAlone = flopTask / (usPerTaskWarm * 1e-6) / 1e12;
    const double tfOff = flopTask / (usPerTaskOff * 1e-6) / 1e12;
    // the k-chunk time at full residency of the kernel with polls off (what
    // the latency is stated against), and of the polled kernel alone
    const double tileUs = usPerTaskOff * blocks / (K / kChunk);
    const double tileUsPolled = usPerTaskWarm * blocks / (K / kChunk);
    printf("\n--- continuous retreat arm: %zu arrivals within the job (%d after it ended, %d "
           "not run), poll %s every %d, %d retreats per arrival, resume %s ---\n",
           raise.size(), afterJob, notRun, pollS.c_str(), pollEvery, retreatBlocks,
           resumeS.c_str());
    if (!raise.empty()) {
      printf("preempt latency, flag raised -> urgent GEMM starts (us): p50 %.2f | p90 %.2f | "
             "p99 %.2f | max %.2f\n", percentile(raise, 0.50), percentile(raise, 0.90),
             percentile(raise, 0.99), *std::max_element(raise.begin(), raise.end()));
      printf("urgent GEMM done after the flag (us): p50 %.2f | p99 %.2f\n",
             percentile(uend, 0.5), percentile(uend, 0.99));
    }
    if (!rfirst.empty())
      printf("retreat after the flag (us): first checkpoint start p50 %.2f | last exit p50 "
             "%.2f p99 %.2f\n", percentile(rfirst, 0.5), percentile(rlast, 0.5),
             percentile(rlast, 0.99));
    if (!cont.empty())
      printf("continuation starts after the flag (us): p50 %.2f | p99 %.2f\n",
             percentile(cont, 0.5), percentile(cont, 0.99));
    printf("tile (k-chunk) time at full residency: %.2f us -> p50 latency = %.3f tiles (polled "
           "kernel: %.2f us -> %.3f)\n", tileUs, raise.empty() ? -1.0 : percentile(raise, 0.5) / tileUs,
           tileUsPolled, raise.empty() ? -1.0 : percentile(raise, 0.5) / tileUsPolled);
    printf("background: %.2f TFLOP/s over the job with arrivals vs %.2f alone (after it) -> retreat "
           "overhead %.2f%%\n", tfJob, tfAlone, (tfAlone / tfJob - 1.0) * 100.0);
    printf("background alone with polls off: %.2f TFLOP/s -> the job with arrivals %.2f%% below "
           "it, the polled kernel alone %.2f%% below it\n", tfOff, (1.0 - tfJob / tfOff) * 100.0,
           (1.0 - tfAlone / tfOff) * 100.0);
    printf("retreats %llu | resumed %llu | save %.2f us per retreat | arrivals without a "
           "retreat %d | late drains %d | resume errors %llu | lost %u | declined (ring full) "
           "%llu | unreleased %u\n", retreats, resumed,
           retreats ? saveTicks * tickUs / retreats : 0.0, noRetreat, lateDrains, errors,
           rr.tail - rr.head, declined, rr.unreleased);
    printf("SAFETY: %lld of %u task fingerprints differ from the unpreempted tile | urgent "
           "outputs not bit-identical: %lld of %d kept\n", hashBad, jobTasks, uBad,
           std::min(events, keepCu + 1));
    if (oracle)
      printf("ORACLE: %s (%lld tasks not executed exactly once)\n",
             oracleBad == 0 ? "PASS" : "FAIL", oracleBad);
    if (csvPath[0]) printf("raw per-arrival records: %s\n", csvPath);
    const bool pass = hashBad == 0 && uBad == 0 && rr.tail == rr.head && errors == 0 &&
                      rr.unclaimed == 0 && rr.unreleased == 0 && oracleBad == 0 &&
                      !raise.empty();
    printf("yield: %s\n", pass ? "PASS" : "FAIL");
    return pass ? 0 : 1;
  }

  if (yieldArm) {
    // --- Retreat arm. Reference fingerprints of every task, unpreempted.
    const std::vector<unsigned long long> refHash = [&] {
      rig.reset(false);
      launch_bg();
      HIP_CHECK(hipStreamSynchronize(bgStream));
      return rig.readTaskHash((unsigned)bgTasks);
    }();
    const std::vector<float> uRefBits = [&] {
      std::vector<float> v((size_t)urgentM * urgentN);
      HIP_CHECK(hipMemcpy(v.data(), dCu, v.size() * 4, hipMemcpyDeviceToHost));
      return v;
    }();
    long long* dRun2;
    unsigned* dExit2;
    HIP_CHECK(hipMalloc(&dRun2, 2 * sizeof(long long)));
    HIP_CHECK(hipMalloc(&dExit2, sizeof(unsigned)));
    // The continuation goes on a third stream ordered after the urgent GEMM by
    // an event: on the urgent stream itself the event the host waits for would
    // only be reported once the continuation (which runs to the end of the
    // job) had finished as well.
    hipEvent_t evU;
    HIP_CHECK(hipEventCreateWithFlags(&evU, hipEventDisableTiming));
    hipStream_t cStream;
    HIP_CHECK(hipStreamCreateWithFlags(&cStream, hipStreamNonBlocking));
    std::mt19937 rng(seed);
    std::uniform_real_distribution<double> frac(0.2, 0.8);
    std::exponential_distribution<double> expo(1.0 / std::max(1.0, meanGapUs));
    struct YRow {
      double delayUs, e2eUs, execUs, gapUs, drainUs, raiseUs, rFirstUs, rLastUs;
      double uEndUs, contUs;  // flag -> urgent GEMM end, flag -> continuation start
      unsigned consumed;
      int retreats;
      std::string placement, retreatXcds;
    };
    std::vector<YRow> rows;
    long long hashBad = 0, oracleBad = 0, uBad = 0, lost = 0;
    int lateDrains = 0, noRetreat = 0;
    unsigned long long retreats = 0, resumed = 0, errors = 0, saveTicks = 0;
    for (int t = 0; t < trials; ++t) {
      rig.reset(false);
      HIP_CHECK(hipMemset(dRun2, 0, 2 * sizeof(long long)));
      HIP_CHECK(hipMemset(dExit2, 0, sizeof(unsigned)));
      HIP_CHECK(hipMemset(dCu, 0xFF, (size_t)urgentM * urgentN * 4));
      HIP_CHECK(hipDeviceSynchronize());
      double delayUs;
      if (arrival == "uniform") {
        delayUs = frac(rng) * drainEstUs;
      } else {
        do delayUs = expo(rng);
        while (delayUs >= 0.95 * drainEstUs);
      }
      const int64_t t0 = now_ns();
      launch_bg();
      spin_until_ns(t0 + (int64_t)(delayUs * 1e3));
      const int64_t tArrive = now_ns();
      HIP_CHECK(hipMemcpyAsync(hConsumed, rig.dNextTask(), APK_QUEUE_XCDS * sizeof(unsigned),
                               hipMemcpyDeviceToHost, uStream));
      APK_CHECK(apk_raise_flag(rig.dFlag(), 1, 1, rig.dSetGT(), uStream));
      launch_urgent();
      HIP_CHECK(hipEventRecord(evU, uStream));
      HIP_CHECK(hipStreamWaitEvent(cStream, evU, 0));
      rig.launchRetreat(poll, pollEvery, resume, (unsigned)bgTasks, retreatN, 1, oracle,
                        retreatBlocks, blocks, true, dRun2, dExit2, cStream);
      HIP_CHECK(hipEventSynchronize(evU));
      const int64_t tDone = now_ns();
      HIP_CHECK(hipStreamSynchronize(cStream));
      HIP_CHECK(hipStreamSynchronize(bgStream));
      RetreatResult rr = rig.readRetreat(1);
      if (rr.tail > rr.head) {
        // A block retreated after the continuation had already drained the
        // queue: relaunch workers until every checkpointed tile is finished.
        ++lateDrains;
        rig.launchRetreat(poll, pollEvery, resume, (unsigned)bgTasks, retreatN, 1, oracle,
                          blocks, blocks + retreatBlocks, true, nullptr, nullptr, bgStream);
        HIP_CHECK(hipStreamSynchronize(bgStream));
        rr = rig.readRetreat(1);
      }
      if (rr.tail != rr.head) lost += rr.tail - rr.head;
      if (rr.unreleased != 0) ++errors;  // an entry claimed but never released
      if (rr.tail == 0) ++noRetreat;
      const EventResult er = rig.readEvents(0);
      for (int b = 0; b < blocks + retreatBlocks; ++b) {
        const unsigned long long* st = &er.stats[(size_t)b * APK_STATS_PER_BLOCK];
        retreats += st[APK_ST_RETREATS];
        resumed += st[APK_ST_RESUMED];
        errors += st[APK_ST_ERRORS];
        saveTicks += st[APK_ST_SAVE];
      }
      const std::vector<unsigned long long> h = rig.readTaskHash((unsigned)bgTasks);
      for (int i = 0; i < bgTasks; ++i) hashBad += h[i] != refHash[i];
      if (oracle) {
        const std::vector<int> ex = rig.readExec((unsigned)bgTasks);
        for (int i = 0; i < bgTasks; ++i) oracleBad += ex[i] != 1;
      }
      std::vector<float> hCu((size_t)urgentM * urgentN);
      HIP_CHECK(hipMemcpy(hCu.data(), dCu, hCu.size() * 4, hipMemcpyDeviceToHost));
      uBad += memcmp(hCu.data(), uRefBits.data(), hCu.size() * 4) != 0;
      auto [bS, bE] = rig.readRunGT();
      long long r2[2];
      HIP_CHECK(hipMemcpy(r2, dRun2, sizeof r2, hipMemcpyDeviceToHost));
      const long long bgEnd = std::max(bE, r2[1]);
      auto [uS, uE] = urgent_window();
      const long long setGT = rr.setGT[0];
      unsigned consumed = 0;
      for (int q = 0; q < APK_QUEUE_XCDS; ++q) consumed += hConsumed[q];
      const bool any = rr.tail > 0;
      rows.push_back({delayUs, (tDone - tArrive) / 1e3, (uE - uS) * tickUs, (uS - bgEnd) * tickUs,
                      (bgEnd - bS) * tickUs, (uS - setGT) * tickUs,
                      any ? (rr.retreatGT[0] - setGT) * tickUs : -1.0,
                      any ? (rr.retreatGT[1] - setGT) * tickUs : -1.0,
                      (uE - setGT) * tickUs, (r2[0] - setGT) * tickUs,
                      std::min(consumed, (unsigned)bgTasks), (int)rr.tail,
                      urgent_placement(), [&] {
                        std::string x;
                        for (int v : rr.xcd) x += (x.empty() ? "" : " ") + std::to_string(v);
                        return x;
                      }()});
    }
    std::vector<double> e2e, raise, rFirst, rLast, exec, drain;
    for (const YRow& r : rows) {
      e2e.push_back(r.e2eUs);
      raise.push_back(r.raiseUs);
      exec.push_back(r.execUs);
      drain.push_back(r.drainUs);
      if (r.retreats > 0) {
        rFirst.push_back(r.rFirstUs);
        rLast.push_back(r.rLastUs);
      }
    }
    printf("\n--- %s, yield on (retreat arm: poll %s every %d, %d retreats per event, resume "
           "%s): %d trials ---\n", mode.c_str(), pollS.c_str(), pollEvery, retreatN,
           resumeS.c_str(), trials);
    printf("urgent e2e (us):  p50 %.1f | p90 %.1f | p99 %.1f | max %.1f\n",
           percentile(e2e, 0.50), percentile(e2e, 0.90), percentile(e2e, 0.99),
           *std::max_element(e2e.begin(), e2e.end()));
    printf("preempt latency, flag raised -> urgent GEMM starts (us): p50 %.2f | p90 %.2f | "
           "p99 %.2f | max %.2f\n", percentile(raise, 0.50), percentile(raise, 0.90),
           percentile(raise, 0.99), *std::max_element(raise.begin(), raise.end()));
    if (!rFirst.empty())
      printf("retreat after the flag (us): first checkpoint start p50 %.2f | last exit p50 "
             "%.2f p99 %.2f\n", percentile(rFirst, 0.5), percentile(rLast, 0.5),
             percentile(rLast, 0.99));
    printf("urgent exec (us): p50 %.2f | p99 %.2f\n", percentile(exec, 0.50),
           percentile(exec, 0.99));
    printf("bg drain (us):    p50 %.0f (no urgent job: %.0f)\n", percentile(drain, 0.50),
           drainEstUs);
    printf("retreats %llu | resumed %llu | save %.2f us per retreat | trials without a "
           "retreat %d | late drains %d | resume errors %llu | lost %lld\n", retreats, resumed,
           retreats ? saveTicks * tickUs / retreats : 0.0, noRetreat, lateDrains, errors, lost);
    printf("SAFETY: %lld of %lld task fingerprints differ from the unpreempted run | urgent "
           "outputs not bit-identical: %lld of %d\n", hashBad, (long long)trials * bgTasks,
           uBad, trials);
    if (oracle)
      printf("ORACLE: %s (%lld tasks not executed exactly once over %d trials)\n",
             oracleBad == 0 ? "PASS" : "FAIL", oracleBad, trials);
    if (csvPath[0]) {
      FILE* csv = fopen(csvPath, "w");
      if (csv) {
        fprintf(csv, "trial,delay_us,consumed_at_arrival,remaining_at_arrival,e2e_us,exec_us,"
                     "gap_us,drain_us,raise_to_ustart_us,retreat_first_us,retreat_last_us,"
                     "retreats,urgent_block_xcd,retreat_xcds,urgent_end_us,cont_start_us\n");
        for (int t = 0; t < trials; ++t)
          fprintf(csv, "%d,%.1f,%u,%d,%.1f,%.2f,%.1f,%.1f,%.2f,%.2f,%.2f,%d,%s,%s,%.2f,%.2f\n", t,
                  rows[t].delayUs, rows[t].consumed, bgTasks - (int)rows[t].consumed,
                  rows[t].e2eUs, rows[t].execUs, rows[t].gapUs, rows[t].drainUs,
                  rows[t].raiseUs, rows[t].rFirstUs, rows[t].rLastUs, rows[t].retreats,
                  rows[t].placement.c_str(), rows[t].retreatXcds.c_str(), rows[t].uEndUs,
                  rows[t].contUs);
        fclose(csv);
        printf("raw trial records: %s\n", csvPath);
      }
    }
    const bool pass = hashBad == 0 && uBad == 0 && lost == 0 && errors == 0 && oracleBad == 0;
    printf("yield: %s\n", pass ? "PASS" : "FAIL");
    return pass ? 0 : 1;
  }

  // --- Trials.
  std::mt19937 rng(seed);
  std::uniform_real_distribution<double> frac(0.2, 0.8);
  std::exponential_distribution<double> expo(1.0 / std::max(1.0, meanGapUs));
  struct Row {
    double delayUs, e2eUs, execUs, gapUs, drainUs;
    unsigned consumed;
  };
  std::vector<Row> rows;
  rows.reserve(trials);
  for (int t = 0; t < trials; ++t) {
    rig.reset(false);
    double delayUs;
    if (arrival == "uniform") {
      delayUs = frac(rng) * drainEstUs;
    } else {
      do delayUs = expo(rng);
      while (delayUs >= 0.95 * drainEstUs);
    }
    const int64_t t0 = now_ns();
    launch_bg();
    spin_until_ns(t0 + (int64_t)(delayUs * 1e3));
    const int64_t tArrive = now_ns();
    HIP_CHECK(hipMemcpyAsync(hConsumed, rig.dNextTask(), APK_QUEUE_XCDS * sizeof(unsigned),
                             hipMemcpyDeviceToHost, uStream));
    launch_urgent();
    HIP_CHECK(hipStreamSynchronize(uStream));
    const int64_t tDone = now_ns();
    HIP_CHECK(hipStreamSynchronize(bgStream));
    auto [bS, bE] = rig.readRunGT();
    auto [uS, uE] = urgent_window();
    unsigned consumed = 0;  // pops handed out at arrival, summed over the XCD lists
    for (int q = 0; q < APK_QUEUE_XCDS; ++q) consumed += hConsumed[q];
    rows.push_back({delayUs, (tDone - tArrive) / 1e3, (uE - uS) * tickUs, (uS - bE) * tickUs,
                    (bE - bS) * tickUs, std::min(consumed, (unsigned)bgTasks)});
  }

  std::vector<double> e2e, gap, exec, drain;
  for (const Row& r : rows) {
    e2e.push_back(r.e2eUs);
    gap.push_back(r.gapUs);
    exec.push_back(r.execUs);
    drain.push_back(r.drainUs);
  }
  printf("\n--- %s: %d trials ---\n", mode.c_str(), trials);
  printf("urgent e2e (us):  p50 %.1f | p90 %.1f | p99 %.1f | max %.1f\n",
         percentile(e2e, 0.50), percentile(e2e, 0.90), percentile(e2e, 0.99),
         *std::max_element(e2e.begin(), e2e.end()));
  printf("gap uStart-bgEnd (us): p50 %.1f | p10 %.1f | p90 %.1f\n", percentile(gap, 0.50),
         percentile(gap, 0.10), percentile(gap, 0.90));
  printf("urgent exec (us): p50 %.2f | p99 %.2f\n", percentile(exec, 0.50),
         percentile(exec, 0.99));
  printf("bg drain (us):    p50 %.0f\n", percentile(drain, 0.50));

  if (csvPath[0]) {
    FILE* csv = fopen(csvPath, "w");
    if (csv) {
      fprintf(csv, "trial,delay_us,consumed_at_arrival,remaining_at_arrival,e2e_us,exec_us,"
                   "gap_us,drain_us\n");
      for (int t = 0; t < trials; ++t)
        fprintf(csv, "%d,%.1f,%u,%d,%.1f,%.2f,%.1f,%.1f\n", t, rows[t].delayUs,
                rows[t].consumed, bgTasks - (int)rows[t].consumed, rows[t].e2eUs,
                rows[t].execUs, rows[t].gapUs, rows[t].drainUs);
      fclose(csv);
      printf("raw trial records: %s\n", csvPath);
    } else {
      fprintf(stderr, "warning: could not open %s\n", csvPath);
    }
  }
  return 0;
}
