// host_selftest -- the measurement binaries' host library (apk_amd/host/
// host_common.cpp) against the CPU oracle (oracle/oracle.cpp) on small,
// ragged inputs, built by tests/native/Makefile with AddressSanitizer and
// UndefinedBehaviorSanitizer (the CPU half of the reference's `make sanitize`,
// Makefile:33-38, whose compute-sanitizer memcheck has no counterpart on this
// GPU pool). Test infrastructure: only tests/test_sanitize.py runs it.
//
// Every check is an exact agreement between two independent implementations:
// glibc-rand inputs, float64 GEMM (whole and by rows, OpenMP and serial),
// elementwise/Frobenius gate, nearest-rank percentile, mt19937 uniform and
// exponential schedules, bf16 round-to-nearest-even (incl. NaN, inf,
// overflow, subnormals, ties), Box-Muller bf16 inputs, bf16 transpose, and the
// argv parser's edge cases (flag as the last word, repeated flags, unknown
// flags, --dtype/--engine agreement). Exit 0 when every check passes.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <cmath>
#include <random>
#include <string>
#include <vector>

#include "host_common.hpp"

extern "C" {
void apko_fill_uniform_pm1(uint32_t seed, float* A, int64_t nA, float* B, int64_t nB);
void apko_gemm_f64(const float* A, const float* B, double* C, int M, int N, int K, int threads);
void apko_gemm_f64_rows(const float* A, const float* B, double* C, int M, int N, int K,
                        int row0, int nrows);
void apko_check_elementwise(const float* got, const double* ref, int64_t n, double rtol,
                            double atol, int64_t* bad, int64_t* nans, double* max_rel);
double apko_rel_frobenius(const float* got, const double* ref, int64_t n);
double apko_percentile(const double* v, int64_t n, double q);
void apko_uniform_gap_schedule(uint32_t seed, double gmin_us, double gmax_us, int events,
                               int64_t* out_cum_ns);
void apko_exp_gap_schedule(uint32_t seed, double mean_us, int events, int64_t* out_cum_ns);
uint16_t apko_bf16_rne(float x);
void apko_fill_normal_bf16(uint32_t seed, uint16_t* A, float* Adeq, int64_t nA, uint16_t* B,
                           float* Bdeq, int64_t nB);
}

namespace {

int failures = 0;
void expect(bool ok, const char* what) {
  if (!ok) {
    ++failures;
    fprintf(stderr, "FAIL: %s\n", what);
  }
}

bool same_bits(const void* a, const void* b, size_t n) { return memcmp(a, b, n) == 0; }

void inputs_and_gemm() {
  const int shapes[][3] = {{1, 1, 1}, {7, 5, 3}, {37, 29, 41}, {64, 48, 17}};
  for (unsigned seed : {0u, 1u, 21u, 977u})
    for (const auto& s : shapes) {
      const int M = s[0], N = s[1], K = s[2];
      std::vector<float> A((size_t)M * K), B((size_t)K * N), Ao(A.size()), Bo(B.size());
      host::fill_uniform_pm1(seed, A, B);
      apko_fill_uniform_pm1(seed, Ao.data(), (int64_t)Ao.size(), Bo.data(), (int64_t)Bo.size());
      expect(same_bits(A.data(), Ao.data(), A.size() * 4) &&
                 same_bits(B.data(), Bo.data(), B.size() * 4),
             "fill_uniform_pm1 agrees with the oracle's glibc restatement");
      std::vector<double> C((size_t)M * N), Co(C.size()), R((size_t)2 * N), Ro(R.size());
      host::gemm_f64(A.data(), B.data(), C.data(), M, N, K, 3);
      apko_gemm_f64(A.data(), B.data(), Co.data(), M, N, K, 1);
      expect(same_bits(C.data(), Co.data(), C.size() * 8), "gemm_f64 (i-k-j) bit-identical");
      const int r0 = M > 2 ? M / 2 : 0, nr = M > 2 ? 2 : 1;
      host::gemm_f64_rows(A.data(), B.data(), R.data(), N, K, r0, nr);
      apko_gemm_f64_rows(A.data(), B.data(), Ro.data(), M, N, K, r0, nr);
      expect(same_bits(R.data(), Ro.data(), (size_t)nr * N * 8), "gemm_f64_rows bit-identical");
      // the gate: perturb a few outputs, compare both checkers
      std::vector<float> got(C.size());
      for (size_t i = 0; i < got.size(); ++i) got[i] = (float)C[i];
      if (got.size() > 3) {
        got[1] += 1e-2f;
        got[got.size() - 1] = NAN;
      }
      const host::CheckResult h = host::check(got.data(), C.data(), (int64_t)C.size(), 1e-4, 1e-4);
      int64_t bad = 0, nans = 0;
      double mr = 0;
      apko_check_elementwise(got.data(), C.data(), (int64_t)C.size(), 1e-4, 1e-4, &bad, &nans, &mr);
      expect(h.bad == bad && h.nans == nans && h.max_rel == mr, "check() agrees elementwise");
      if (nans == 0)
        expect(std::fabs(h.rel_frob - apko_rel_frobenius(got.data(), C.data(),
                                                        (int64_t)C.size())) <=
                   1e-12 * (1 + h.rel_frob),
               "check() rel-Frobenius agrees");
    }
}

void percentiles_and_schedules() {
  std::mt19937 g(5);
  for (int n : {1, 2, 3, 10, 101, 1000}) {
    std::vector<double> v(n);
    for (auto& x : v) x = (double)(g() % 1000) / 7.0;
    for (double q : {0.0, 0.01, 0.5, 0.9, 0.99, 0.999, 1.0})
      expect(host::percentile(v, q) == apko_percentile(v.data(), n, q),
             "nearest-rank percentile agrees");
  }
  expect(std::isnan(host::percentile({}, 0.5)), "percentile of nothing is NaN");
  for (unsigned seed : {1u, 21u, 12345u})
    for (int ev : {1, 17, 1000}) {
      const std::vector<long long> u = host::uniform_schedule(seed, 150, 400, ev);
      const std::vector<long long> e = host::exp_schedule(seed, 2000, ev);
      std::vector<int64_t> uo(ev), eo(ev);
      apko_uniform_gap_schedule(seed, 150, 400, ev, uo.data());
      apko_exp_gap_schedule(seed, 2000, ev, eo.data());
      bool ok = true;
      for (int i = 0; i < ev; ++i) ok = ok && u[i] == uo[i] && e[i] == eo[i];
      expect(ok, "uniform and exponential schedules agree with the mt19937 restatement");
    }
}

void bf16() {
  std::vector<float> xs = {0.0f, -0.0f, 1.0f, -1.0f, 3.4028235e38f, -3.4028235e38f,
                           1e-45f, -1e-45f, 1.17549435e-38f, INFINITY, -INFINITY, NAN};
  // ties: bf16 keeps 7 mantissa bits; 1 + 2^-8 is halfway between 1 and 1 + 2^-7
  for (uint32_t u : {0x3f808000u, 0x3f818000u, 0x3f80c000u, 0x7f7f8000u, 0x00008000u,
                     0x80018000u, 0x7f800001u, 0xffc00001u}) {
    float f;
    memcpy(&f, &u, 4);
    xs.push_back(f);
  }
  std::mt19937 g(9);
  for (int i = 0; i < 100000; ++i) {
    const uint32_t u = g();
    float f;
    memcpy(&f, &u, 4);
    xs.push_back(f);
  }
  // NaN inputs: both give a quiet bf16 NaN (the host library a canonical
  // one, the oracle the input's sign and top payload bits); the generated
  // inputs never hold a NaN.
  auto isnan16 = [](uint16_t h) { return (h & 0x7f80u) == 0x7f80u && (h & 0x007fu) != 0; };
  bool ok = true;
  for (float x : xs)
    ok = ok && (std::isnan(x) ? isnan16(host::bf16_rne(x)) && isnan16(apko_bf16_rne(x))
                              : host::bf16_rne(x) == apko_bf16_rne(x));
  expect(ok, "bf16 round-to-nearest-even agrees (NaN, inf, overflow, ties, subnormals)");
  for (unsigned seed : {0u, 21u}) {
    const int nA = 37 * 29, nB = 29 * 41;
    std::vector<float> A(nA), B(nB), Ao(nA), Bo(nB);
    std::vector<uint16_t> Ab, Bb, Abo(nA), Bbo(nB);
    host::fill_normal_bf16(seed, A, Ab, B, Bb);
    apko_fill_normal_bf16(seed, Abo.data(), Ao.data(), nA, Bbo.data(), Bo.data(), nB);
    expect(Ab == Abo && Bb == Bbo && same_bits(A.data(), Ao.data(), nA * 4) &&
               same_bits(B.data(), Bo.data(), nB * 4),
           "Box-Muller bf16 inputs agree");
    const std::vector<uint16_t> T = host::transpose_u16(Ab, 37, 29);
    bool tok = T.size() == Ab.size();
    for (int r = 0; r < 37 && tok; ++r)
      for (int c = 0; c < 29; ++c) tok = tok && T[(size_t)c * 37 + r] == Ab[(size_t)r * 29 + c];
    expect(tok, "transpose_u16");
  }
}

void argv_parsing() {
  auto mk = [](std::vector<std::string>& words) {
    std::vector<char*> v;
    for (auto& w : words) v.push_back(&w[0]);
    return v;
  };
  std::vector<std::string> w = {"bin", "--k", "64", "--unknown", "7", "--k", "128", "--csv"};
  std::vector<char*> a = mk(w);
  const int argc = (int)a.size();
  expect(host::parse_arg(argc, a.data(), "--k", 1) == 64, "first match wins");
  expect(host::parse_arg(argc, a.data(), "--blocks", 5) == 5, "absent flag keeps its default");
  // a flag as the last word has no value: the default stands, nothing is read past argv
  expect(host::parse_arg(argc, a.data(), "--csv", 3) == 3, "flag without a value");
  expect(std::string(host::parse_str(argc, a.data(), "--csv", "d")) == "d", "string flag without a value");
  std::vector<std::string> e1 = {"bin", "--dtype", "bf16"}, e2 = {"bin", "--engine", "bf16x128"},
                           e3 = {"bin", "--dtype", "fp32", "--engine", "bf16x256"},
                           e4 = {"bin", "--dtype", "f64"};
  std::vector<char*> a1 = mk(e1), a2 = mk(e2), a3 = mk(e3), a4 = mk(e4);
  expect(host::engine_arg(3, a1.data(), "mfma128") == "bf16x256", "--dtype bf16");
  expect(host::engine_arg(3, a2.data(), "mfma128") == "bf16x128", "--engine alone");
  expect(host::engine_arg(5, a3.data(), "mfma128").empty(), "--dtype and --engine disagree");
  expect(host::engine_arg(3, a4.data(), "mfma128").empty(), "unknown --dtype");
  expect(host::engine_arg(1, a1.data(), "mfma128") == "mfma128", "fp32 default");
}

}  // namespace

int main() {
  inputs_and_gemm();
  percentiles_and_schedules();
  bf16();
  argv_parsing();
  printf("%s host_selftest: %d failed checks\n", failures ? "FAIL" : "PASS", failures);
  return failures ? 1 : 0;
}
