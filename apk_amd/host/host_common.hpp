// host_common.hpp -- host-side harness shared by the measurement binaries:
// the reference's CLI conventions, input generation, float64 verification,
// nearest-rank statistics, schedules and CSV output, in plain C++ over the
// HIP runtime and the apk C ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "apk.h"

// HIP_CHECK / APK_CHECK print "HIP error at file:line: msg" and exit(1), the
// reference's CUDA_CHECK contract (src/persistent.cu:41-49).
#define HIP_CHECK(call)                                                   \
  do {                                                                    \
    hipError_t err_ = (call);                                             \
    if (err_ != hipSuccess) {                                             \
      fprintf(stderr, "HIP error at %s:%d: %s\n", __FILE__, __LINE__,     \
              hipGetErrorString(err_));                                   \
      exit(1);                                                            \
    }                                                                     \
  } while (0)

#define APK_CHECK(call)                                                   \
  do {                                                                    \
    int rc_ = (call);                                                     \
    if (rc_ != APK_OK) {                                                  \
      fprintf(stderr, "apk error at %s:%d: %s\n", __FILE__, __LINE__,     \
              apk_last_error());                                          \
      exit(1);                                                            \
    }                                                                     \
  } while (0)

namespace host {

// argv linear scan, first match wins, unknown flags ignored, numbers via
// atof (src/persistent.cu:83-94).
double parse_arg(int argc, char** argv, const char* name, double dflt);
const char* parse_str(int argc, char** argv, const char* name, const char* dflt);
// The tile engine named by --engine, or chosen by --dtype fp32|bf16 when
// --engine is absent (fp32: `fp32Default`; bf16: bf16x256). Returns "" when
// the two flags disagree or --dtype is neither, which the caller reports as a
// bad flag.
std::string engine_arg(int argc, char** argv, const char* fp32Default);

int64_t now_ns();
void spin_for_ns(int64_t ns);
void spin_until_ns(int64_t deadline);

// Nearest-rank percentile v[min(int(q*n), n-1)] of a sorted copy
// (src/yield.cu:322-325).
double percentile(std::vector<double> v, double q);

// glibc srand(seed); rand()/RAND_MAX*2-1 for A (M*K) then B (K*N)
// (src/persistent.cu:131-135). glibc treats seed 0 as seed 1.
void fill_uniform_pm1(unsigned seed, std::vector<float>& A, std::vector<float>& B);

// normal(0,1) values rounded to bf16 (round to nearest even): Box-Muller
// over std::mt19937(seed) with std::generate_canonical<double, 53> draws
// (u1 = 1 - u in (0,1], u2 in [0,1)), both outputs of each pair used, A
// first then B; *_bits gets the bf16 bit patterns, A/B (sized by the caller)
// the exact float values they encode (what the float64 reference
// multiplies, as src/tcyield.cu:459-473 does for its fp16 data).
void fill_normal_bf16(unsigned seed, std::vector<float>& A, std::vector<uint16_t>& A_bits,
                      std::vector<float>& B, std::vector<uint16_t>& B_bits);
uint16_t bf16_rne(float x);
// rows x cols -> cols x rows.
std::vector<uint16_t> transpose_u16(const std::vector<uint16_t>& m, int rows, int cols);
template <class T>
std::vector<uint8_t> as_bytes(const std::vector<T>& v) {
  const uint8_t* p = reinterpret_cast<const uint8_t*>(v.data());
  return std::vector<uint8_t>(p, p + v.size() * sizeof(T));
}

// float64 reference C = A.B (row-major), i-k-j order with double
// accumulation per element (src/persistent.cu:221-227); rows are split over
// OpenMP threads, which does not change any element's summation order.
void gemm_f64(const float* A, const float* B, double* C, int M, int N, int K,
              int threads);
// Rows [r0, r0+nr) only, into C (nr x N).
void gemm_f64_rows(const float* A, const float* B, double* C, int N, int K,
                   int r0, int nr);

struct CheckResult {
  int64_t bad = 0, nans = 0;
  double max_rel = 0.0;  // err / max(1, |ref|)
  double rel_frob = 0.0; // ||got-ref||_F / ||ref||_F
};
// Elementwise gate |got-ref| <= atol + rtol*|ref| (src/persistent.cu:228-237)
// plus the relative Frobenius error.
CheckResult check(const float* got, const double* ref, int64_t n, double rtol,
                  double atol);

// Device description line + values used for unit conversion.
struct Device {
  apk_device_info info;
  double wall_mhz;  // device wall clock in MHz (ticks per us)
};
Device device_query();

// Engine clock beside a throughput figure: one-wave apk_clock_probe blocks
// on a stream of their own, launched right after the kernel they time and
// counting shader cycles against the wall clock over `window_us`. The
// stream is created and warmed by the constructor, so the first timed
// launch does not wait for its queue. read() after the device has synced.
class ClockProbe {
 public:
  explicit ClockProbe(int probes = 32);
  ~ClockProbe();
  void launch(double window_us, double wall_mhz);
  // mean / min / max MHz over the probes that ran, and only those whose
  // window lies inside [lo, hi] wall ticks when hi > 0; false when none did.
  bool read(double wall_mhz, double* mean, double* mn, double* mx, int* n,
            long long lo = 0, long long hi = 0) const;
  // "engine clock during <what> (N probes): mean X MHz | min | max"
  void print(const char* what, double wall_mhz, long long lo = 0, long long hi = 0) const;

 private:
  int probes_;
  long long* d_ = nullptr;
  hipStream_t s_ = nullptr;
};

// Event schedules (cumulative ns). uniform: mt19937(seed), U(gmin,gmax) us,
// truncated per gap (src/yield.cu:824-830). exponential: mean_us.
std::vector<long long> uniform_schedule(unsigned seed, double gmin_us,
                                        double gmax_us, int events);
std::vector<long long> exp_schedule(unsigned seed, double mean_us, int events);

// FLOP/s and byte figures.
inline double tflops(double flop, double seconds) { return flop / seconds / 1e12; }

// MI355X published peaks used as roofline denominators.
constexpr double kPeakFp32TF = 157.3;    // fp32 matrix (and vector FMA) dense
constexpr double kPeakBf16TF = 2516.6;   // bf16 MFMA dense
constexpr double kPeakHbmGBs = 8000.0;   // HBM3E

}  // namespace host
