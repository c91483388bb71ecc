// host_common.cpp -- see host_common.hpp.
#include "host_common.hpp"

#include <omp.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <random>

namespace host {

double parse_arg(int argc, char** argv, const char* name, double dflt) {
  for (int i = 1; i + 1 < argc; ++i)
    if (strcmp(argv[i], name) == 0) return atof(argv[i + 1]);
  return dflt;
}

const char* parse_str(int argc, char** argv, const char* name, const char* dflt) {
  for (int i = 1; i + 1 < argc; ++i)
    if (strcmp(argv[i], name) == 0) return argv[i + 1];
  return dflt;
}

std::string engine_arg(int argc, char** argv, const char* fp32Default) {
  const std::string eng = parse_str(argc, argv, "--engine", "");
  const std::string dt = parse_str(argc, argv, "--dtype", "");
  const bool engBf16 = eng.rfind("bf16", 0) == 0;
  if (dt.empty()) return eng.empty() ? std::string(fp32Default) : eng;
  if (dt == "bf16" && (eng.empty() || engBf16)) return eng.empty() ? "bf16x256" : eng;
  if ((dt == "fp32" || dt == "f32") && (eng.empty() || !engBf16))
    return eng.empty() ? std::string(fp32Default) : eng;
  fprintf(stderr, "--dtype %s does not name the operand type of --engine %s (fp32|bf16)\n",
          dt.c_str(), eng.empty() ? "(none)" : eng.c_str());
  return "";
}

int64_t now_ns() {
  using namespace std::chrono;
  return duration_cast<nanoseconds>(steady_clock::now().time_since_epoch()).count();
}

void spin_until_ns(int64_t deadline) {
  while (now_ns() < deadline) {
  }
}

void spin_for_ns(int64_t ns) { spin_until_ns(now_ns() + ns); }

double percentile(std::vector<double> v, double q) {
  if (v.empty()) return NAN;
  std::sort(v.begin(), v.end());
  return v[std::min((size_t)(q * v.size()), v.size() - 1)];
}

void fill_uniform_pm1(unsigned seed, std::vector<float>& A, std::vector<float>& B) {
  srand(seed);
  for (auto& v : A) v = (float)(rand() / (double)RAND_MAX * 2.0 - 1.0);
  for (auto& v : B) v = (float)(rand() / (double)RAND_MAX * 2.0 - 1.0);
}

void gemm_f64_rows(const float* A, const float* B, double* C, int N, int K,
                   int r0, int nr) {
  for (int ii = 0; ii < nr; ++ii) {
    const int i = r0 + ii;
    double* crow = C + (size_t)ii * N;
    std::fill(crow, crow + N, 0.0);
    for (int k = 0; k < K; ++k) {
      const double a = A[(size_t)i * K + k];
      const float* brow = B + (size_t)k * N;
      for (int j = 0; j < N; ++j) crow[j] += a * brow[j];
    }
  }
}

void gemm_f64(const float* A, const float* B, double* C, int M, int N, int K,
              int threads) {
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 4) num_threads(threads)
  for (int i = 0; i < M; ++i) gemm_f64_rows(A, B, C + (size_t)i * N, N, K, i, 1);
}

CheckResult check(const float* got, const double* ref, int64_t n, double rtol,
                  double atol) {
  CheckResult r;
  long double num = 0, den = 0;
  for (int64_t i = 0; i < n; ++i) {
    den += (long double)ref[i] * ref[i];
    if (std::isnan(got[i])) {
      ++r.nans;
      continue;
    }
    const double err = std::fabs((double)got[i] - ref[i]);
    num += (long double)err * err;
    r.max_rel = std::max(r.max_rel, err / std::max(1.0, std::fabs(ref[i])));
    if (err > atol + rtol * std::fabs(ref[i])) ++r.bad;
  }
  r.rel_frob = den > 0 ? (double)std::sqrt(num / den) : (num > 0 ? INFINITY : 0.0);
  if (r.nans) r.rel_frob = NAN;
  return r;
}

Device device_query() {
  Device d;
  APK_CHECK(apk_get_device_info(0, &d.info));
  d.wall_mhz = d.info.wall_clock_khz / 1000.0;
  return d;
}

ClockProbe::ClockProbe(int probes) : probes_(probes) {
  HIP_CHECK(hipMalloc(&d_, (size_t)probes_ * 4 * sizeof(long long)));
  HIP_CHECK(hipMemset(d_, 0, (size_t)probes_ * 4 * sizeof(long long)));
  HIP_CHECK(hipStreamCreateWithFlags(&s_, hipStreamNonBlocking));
  APK_CHECK(apk_clock_probe(d_, probes_, 1, s_));  // creates the stream's queue
  HIP_CHECK(hipStreamSynchronize(s_));
  HIP_CHECK(hipMemset(d_, 0, (size_t)probes_ * 4 * sizeof(long long)));
}

ClockProbe::~ClockProbe() {
  (void)hipStreamSynchronize(s_);
  (void)hipStreamDestroy(s_);
  (void)hipFree(d_);
}

void ClockProbe::launch(double window_us, double wall_mhz) {
  const long long w = std::max(1LL, (long long)(window_us * wall_mhz));
  APK_CHECK(apk_clock_probe(d_, probes_, std::min(w, 6000000000LL), s_));
}

bool ClockProbe::read(double wall_mhz, double* mean, double* mn, double* mx, int* count,
                      long long lo_t, long long hi_t) const {
  std::vector<long long> pr((size_t)probes_ * 4);
  HIP_CHECK(hipMemcpy(pr.data(), d_, pr.size() * sizeof(long long), hipMemcpyDeviceToHost));
  double sum = 0, lo = 0, hi = 0;
  int n = 0;
  for (int i = 0; i < probes_; ++i) {
    if (pr[4 * i + 1] <= 0) continue;
    if (hi_t > 0 && (pr[4 * i + 3] < lo_t || pr[4 * i + 3] + pr[4 * i + 1] > hi_t)) continue;
    const double mhz = (double)pr[4 * i] / (double)pr[4 * i + 1] * wall_mhz;
    lo = n ? std::min(lo, mhz) : mhz;
    hi = n ? std::max(hi, mhz) : mhz;
    sum += mhz;
    ++n;
  }
  *count = n;
  if (!n) return false;
  *mean = sum / n;
  *mn = lo;
  *mx = hi;
  return true;
}

void ClockProbe::print(const char* what, double wall_mhz, long long lo, long long hi) const {
  double mean, mn, mx;
  int n = 0;
  if (read(wall_mhz, &mean, &mn, &mx, &n, lo, hi))
    printf("engine clock during %s (%d probes): mean %.0f MHz | min %.0f | max %.0f\n", what,
           n, mean, mn, mx);
  else
    printf("engine clock during %s: no probe ran inside it\n", what);
}

std::vector<long long> uniform_schedule(unsigned seed, double gmin_us,
                                        double gmax_us, int events) {
  std::mt19937 rng(seed);
  std::uniform_real_distribution<double> gap(gmin_us * 1000.0, gmax_us * 1000.0);
  std::vector<long long> out(std::max(events, 1), 0);
  long long acc = 0;
  for (int e = 0; e < events; ++e) out[e] = (acc += (long long)gap(rng));
  return out;
}

std::vector<long long> exp_schedule(unsigned seed, double mean_us, int events) {
  std::mt19937 rng(seed);
  std::exponential_distribution<double> gap(1.0 / (mean_us * 1000.0));
  std::vector<long long> out(std::max(events, 1), 0);
  long long acc = 0;
  for (int e = 0; e < events; ++e) out[e] = (acc += (long long)gap(rng));
  return out;
}

}  // namespace host

namespace host {

uint16_t bf16_rne(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return 0x7fc0;  // NaN
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

void fill_normal_bf16(unsigned seed, std::vector<float>& A, std::vector<uint16_t>& A_bits,
                      std::vector<float>& B, std::vector<uint16_t>& B_bits) {
  std::mt19937 g(seed);
  const double two_pi = 6.283185307179586476925286766559;
  bool have = false;
  double spare = 0.0;
  auto next = [&]() -> float {
    if (have) {
      have = false;
      return (float)spare;
    }
    const double u1 = 1.0 - std::generate_canonical<double, 53>(g);
    const double u2 = std::generate_canonical<double, 53>(g);
    const double r = std::sqrt(-2.0 * std::log(u1));
    spare = r * std::sin(two_pi * u2);
    have = true;
    return (float)(r * std::cos(two_pi * u2));
  };
  auto fill = [&](std::vector<float>& v, std::vector<uint16_t>& bits) {
    bits.resize(v.size());
    for (size_t i = 0; i < v.size(); ++i) {
      bits[i] = bf16_rne(next());
      const uint32_t u = (uint32_t)bits[i] << 16;
      memcpy(&v[i], &u, 4);
    }
  };
  fill(A, A_bits);
  fill(B, B_bits);
}

std::vector<uint16_t> transpose_u16(const std::vector<uint16_t>& m, int rows, int cols) {
  std::vector<uint16_t> t(m.size());
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < cols; ++c) t[(size_t)c * rows + r] = m[(size_t)r * cols + c];
  return t;
}

}  // namespace host
