// capi_common.hip -- device queries and error reporting of the C ABI.
#include <stdarg.h>
#include <string.h>
#include "capi.hpp"
#include "engine_bf16.hpp"
#include "engine_mfma128.hpp"
#include "engine_valu64.hpp"

namespace apk {
static thread_local char g_err[512] = "";
void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}
}  // namespace apk

extern "C" const char* apk_last_error(void) { return apk::g_err; }

extern "C" int apk_get_device_info(int device, apk_device_info* out) {
  APK_REQUIRE(out != nullptr, "apk_get_device_info: out is NULL");
  hipDeviceProp_t p;
  APK_HIP(hipGetDeviceProperties(&p, device));
  memset(out, 0, sizeof *out);
  strncpy(out->name, p.name, sizeof out->name - 1);
  strncpy(out->arch, p.gcnArchName, sizeof out->arch - 1);
  out->cu_count = p.multiProcessorCount;
  int wc = 0;
  APK_HIP(hipDeviceGetAttribute(&wc, hipDeviceAttributeWallClockRate, device));
  out->wall_clock_khz = wc;
  out->clock_khz = p.clockRate;
  out->lds_per_cu = (int)p.maxSharedMemoryPerMultiProcessor;
  out->regs_per_cu = p.regsPerMultiprocessor;
  // gfx950 has 32 CUs per XCD (8 XCDs x 32 = 256 CUs).
  out->xcc_count = p.multiProcessorCount >= 32 ? p.multiProcessorCount / 32 : 1;
  return APK_OK;
}

extern "C" int apk_engine_geometry_of(int engine, apk_engine_geometry* out) {
  APK_REQUIRE(out != nullptr, "apk_engine_geometry_of: out is NULL");
  switch (engine) {
    case APK_ENGINE_VALU64:
      *out = {apk::EngValu64::TM, apk::EngValu64::TN, apk::EngValu64::KS,
              apk::EngValu64::THREADS, apk::EngValu64::LDS_BYTES, 4, 0};
      return APK_OK;
    case APK_ENGINE_MFMA128:
      *out = {apk::EngMfma128::TM, apk::EngMfma128::TN, apk::EngMfma128::KS,
              apk::EngMfma128::THREADS, apk::EngMfma128::LDS_BYTES, 4, 0};
      return APK_OK;
    case APK_ENGINE_BF16X256:
      *out = {apk::EngBf16x256::TM, apk::EngBf16x256::TN, apk::EngBf16x256::KS,
              apk::EngBf16x256::THREADS, apk::EngBf16x256::LDS_BYTES, 2, 1};
      return APK_OK;
    case APK_ENGINE_BF16X128:
      *out = {apk::EngBf16x128::TM, apk::EngBf16x128::TN, apk::EngBf16x128::KS,
              apk::EngBf16x128::THREADS, apk::EngBf16x128::LDS_BYTES, 2, 1};
      return APK_OK;
    case APK_ENGINE_BF16X256X128:
      *out = {apk::EngBf16x256x128::TM, apk::EngBf16x256x128::TN, apk::EngBf16x256x128::KS,
              apk::EngBf16x256x128::THREADS, apk::EngBf16x256x128::LDS_BYTES, 2, 1};
      return APK_OK;
    default:
      apk::set_error("unknown engine %d", engine);
      return APK_EINVAL;
  }
}
