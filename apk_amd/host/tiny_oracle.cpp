// tiny_oracle.cpp -- see tiny_oracle.hpp. Host side of the exactly-once
// scheduler oracle on tiny tasks (apk_tiny_oracle).
#include "tiny_oracle.hpp"

#include <omp.h>

#include <algorithm>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "host_common.hpp"

namespace host {
namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;
constexpr uint64_t kUrgentSalt = 0xD1B54A32D192ED03ull;

uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

float bf16_value(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Fingerprint of the product of A tile ia and B tile ib (Bt stored N x K),
// taken in the device's register order: position p = 4 l + j holds
// C[4 (l / 16) + j][l % 16]. Small-integer operands: every value is exact.
uint64_t tile_value(const std::vector<uint16_t>& A, const std::vector<uint16_t>& Bt, int ia,
                    int ib) {
  uint64_t v = 0;
  for (int l = 0; l < 64; ++l)
    for (int j = 0; j < 4; ++j) {
      const int row = 4 * (l / 16) + j, col = l % 16;
      float acc = 0.f;
      for (int k = 0; k < 16; ++k)
        acc += bf16_value(A[(size_t)ia * 256 + row * 16 + k]) *
               bf16_value(Bt[(size_t)ib * 256 + col * 16 + k]);
      uint32_t bits;
      std::memcpy(&bits, &acc, 4);
      v += mix64((uint64_t)bits + ((uint64_t)(4 * l + j) << 32));
    }
  return v;
}

// Small integers in [-2, 2] as bf16 bit patterns (exact), mt19937(seed).
std::vector<uint16_t> small_int_tiles(unsigned seed, int tiles) {
  std::mt19937 g(seed);
  std::vector<uint16_t> out((size_t)tiles * 256);
  for (auto& x : out) {
    const float v = (float)((int)(g() % 5u) - 2);
    uint32_t u;
    std::memcpy(&u, &v, 4);
    x = (uint16_t)(u >> 16);
  }
  return out;
}

}  // namespace

int run_tiny_oracle(int argc, char** argv) {
  const double tasksD = parse_arg(argc, argv, "--tasks", 1e8);
  const int batch = (int)parse_arg(argc, argv, "--tiny-batch", 1);
  const int events = (int)parse_arg(argc, argv, "--events", 1000);
  const double meanGapUs = parse_arg(argc, argv, "--mean-gap-us", 50);
  const int U = (int)parse_arg(argc, argv, "--urgent-tiles", 64);
  const int pa = (int)parse_arg(argc, argv, "--pa", 64);
  const int pb = (int)parse_arg(argc, argv, "--pb", 64);
  const int bpc = (int)parse_arg(argc, argv, "--blocks-per-cu", 2);
  const unsigned seed = (unsigned)parse_arg(argc, argv, "--seed", 21);
  if (tasksD < 1 || tasksD > 4.0e9 || batch < 1 || events < 0 || U < 0 || pa < 1 || pb < 1 ||
      bpc < 1) {
    fprintf(stderr, "bad --tasks (1..4e9), --tiny-batch, --events, --urgent-tiles, --pa/--pb "
            "or --blocks-per-cu\n");
    return 1;
  }
  const unsigned N = (unsigned)tasksD;
  const Device dev = device_query();
  const int blocks = dev.info.cu_count * bpc;
  const int waves = blocks * 4;
  printf("GPU: %s | %d CUs | tiny-task oracle: %u tasks of 16x16x16 bf16 MFMA, %d waves "
         "(%d blocks/CU x 4), batch %d | %d events, exponential gaps mean %.0f us, %d urgent "
         "tasks each\n", dev.info.arch, dev.info.cu_count, N, waves, bpc, batch, events,
         meanGapUs, U);

  const std::vector<uint16_t> A = small_int_tiles(seed, pa);
  const std::vector<uint16_t> Bt = small_int_tiles(seed + 1, pb);
  const std::vector<long long> gapsNs = events ? exp_schedule(seed, meanGapUs, events)
                                               : std::vector<long long>();
  std::vector<long long> sched(std::max(events, 1), 0);
  for (int e = 0; e < events; ++e) sched[e] = (long long)(gapsNs[e] * dev.wall_mhz / 1000.0);

  auto dalloc = [](size_t bytes) {
    void* p = nullptr;
    HIP_CHECK(hipMalloc(&p, std::max<size_t>(bytes, 64)));
    HIP_CHECK(hipMemset(p, 0, std::max<size_t>(bytes, 64)));
    return p;
  };
  const int E = std::max(events, 1);
  auto* dA = (uint16_t*)dalloc(A.size() * 2);
  auto* dBt = (uint16_t*)dalloc(Bt.size() * 2);
  auto* dNext = (unsigned*)dalloc(APK_QUEUE_WORDS * 4);
  auto* dExec = (int*)dalloc((size_t)N * 4);
  auto* dSum = (unsigned long long*)dalloc(16);
  auto* dFlag = (int*)dalloc(64);
  auto* dSched = (long long*)dalloc((size_t)E * 8);
  auto* dSet = (long long*)dalloc((size_t)E * 8);
  auto* dUq = (int*)dalloc((size_t)E * 4);
  auto* dUexec = (int*)dalloc((size_t)E * 4);
  auto* dCkpt = (float*)dalloc((size_t)waves * 256 * 4);
  auto* dStats = (unsigned long long*)dalloc(16);
  HIP_CHECK(hipMemcpy(dA, A.data(), A.size() * 2, hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(dBt, Bt.data(), Bt.size() * 2, hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(dSched, sched.data(), sched.size() * 8, hipMemcpyHostToDevice));

  apk_tiny_params p;
  std::memset(&p, 0, sizeof p);
  p.num_tasks = N;
  p.next_task = dNext;
  p.batch = batch;
  p.A = dA;
  p.Bt = dBt;
  p.pa = pa;
  p.pb = pb;
  p.exec_count = dExec;
  p.checksum = dSum;
  p.flag = dFlag;
  if (events) {
    p.sched = dSched;
    p.num_events = events;
    p.set_gt = dSet;
    p.uq_next = dUq;
    p.urgent_per_event = U;
    p.u_exec_count = dUexec;
  }
  p.ckpt = dCkpt;
  p.stats = dStats;

  hipStream_t st;
  HIP_CHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  hipEvent_t e0, e1;
  HIP_CHECK(hipEventCreate(&e0));
  HIP_CHECK(hipEventCreate(&e1));
  HIP_CHECK(hipDeviceSynchronize());
  HIP_CHECK(hipEventRecord(e0, st));
  APK_CHECK(apk_tiny_oracle(&p, blocks, st));
  HIP_CHECK(hipEventRecord(e1, st));
  HIP_CHECK(hipStreamSynchronize(st));
  HIP_CHECK(hipGetLastError());
  float ms = 0;
  HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));

  // Exactly-once: every task counted once.
  std::vector<int> ex(N);
  HIP_CHECK(hipMemcpy(ex.data(), dExec, (size_t)N * 4, hipMemcpyDeviceToHost));
  long long dup = 0, missed = 0, firstBad = -1;
#pragma omp parallel for reduction(+ : dup, missed) schedule(static)
  for (long long t = 0; t < (long long)N; ++t) {
    if (ex[t] > 1) ++dup;
    if (ex[t] < 1) ++missed;
  }
  if (dup || missed)
    for (long long t = 0; t < (long long)N; ++t)
      if (ex[t] != 1) {
        firstBad = t;
        break;
      }
  std::vector<long long> set(E);
  std::vector<int> uex(E);
  unsigned long long sum[2], stats[2];
  HIP_CHECK(hipMemcpy(set.data(), dSet, (size_t)E * 8, hipMemcpyDeviceToHost));
  HIP_CHECK(hipMemcpy(uex.data(), dUexec, (size_t)E * 4, hipMemcpyDeviceToHost));
  HIP_CHECK(hipMemcpy(sum, dSum, 16, hipMemcpyDeviceToHost));
  HIP_CHECK(hipMemcpy(stats, dStats, 16, hipMemcpyDeviceToHost));
  int fired = 0, badU = 0;
  for (int e = 0; e < events; ++e) {
    if (set[e] != 0) {
      ++fired;
      if (uex[e] != U) ++badU;
    } else if (uex[e] != 0) {
      ++badU;
    }
  }

  // Predicted checksums: tile fingerprints per (A, B) pair, then the sums.
  const int threads = (int)std::max(1u, std::thread::hardware_concurrency());
  std::vector<uint64_t> V((size_t)pa * pb);
#pragma omp parallel for num_threads(threads) schedule(dynamic)
  for (int i = 0; i < pa * pb; ++i) V[i] = tile_value(A, Bt, i % pa, i / pa);
  uint64_t wantBg = 0;
#pragma omp parallel for num_threads(threads) reduction(+ : wantBg) schedule(static)
  for (long long t = 0; t < (long long)N; ++t)
    wantBg += mix64(V[(size_t)(((uint64_t)t / pa) % pb) * pa + (uint64_t)t % pa] +
                    (uint64_t)t * kGolden);
  uint64_t wantU = 0;
  const uint64_t nU = (uint64_t)fired * (uint64_t)U;
  for (uint64_t id = 0; id < nU; ++id)
    wantU += mix64(V[(size_t)((id * 13 + 5) % pb) * pa + (id * 7 + 3) % pa] + id * kGolden +
                   kUrgentSalt);

  printf("run: %.3f ms -> %.1f M tasks/s (%.1f ns per task per wave)\n", ms, N / (ms * 1e3),
         ms * 1e6 * waves / N);
  printf("events: %d of %d fired | yields %llu | urgent tasks %llu (want %llu)\n", fired, events,
         stats[0], stats[1], (unsigned long long)nU);
  printf("oracle tasks: %u checked | duplicates %lld | missed %lld", N, dup, missed);
  if (firstBad >= 0) printf(" | first bad %lld (count %d)", firstBad, ex[firstBad]);
  printf("\noracle events: urgent-count violations %d\n", badU);
  printf("checksums: background %s, urgent %s\n", sum[0] == wantBg ? "match" : "DIFFER",
         sum[1] == wantU ? "match" : "DIFFER");
  const bool pass = dup == 0 && missed == 0 && badU == 0 && fired == events &&
                    stats[1] == nU && sum[0] == wantBg && sum[1] == wantU;
  printf("ORACLE: %s\n", pass ? "PASS" : "FAIL");
  return pass ? 0 : 1;
}

}  // namespace host
