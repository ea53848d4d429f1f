// Library-wide C-ABI helpers: version, last error, device limits.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <string>

#include "tw_capi.hpp"
#include "../../include/torchwarp_hip.h"

namespace {
thread_local std::string g_last_error;
std::once_flag g_lds_once[64];
int g_lds_bytes[64];
std::once_flag g_clk_once[64];
int g_clk_khz[64];
std::once_flag g_cu_once[64];
int g_cus[64];
}  // namespace

namespace tw {

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(TW_ELAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  }
  return TW_OK;
}

int max_lds_bytes() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 64 * 1024;
  std::call_once(g_lds_once[dev], [dev] {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
        v <= 0) {
      v = 64 * 1024;
    }
    g_lds_bytes[dev] = v;
  });
  return g_lds_bytes[dev];
}

int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::call_once(g_cu_once[dev], [dev] {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        v <= 0)
      v = 256;
    g_cus[dev] = v;
  });
  return g_cus[dev];
}

double realtime_khz() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 100000.0;
  std::call_once(g_clk_once[dev], [dev] {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeWallClockRate, dev) != hipSuccess || v <= 0)
      v = 100000;   // 100 MHz
    g_clk_khz[dev] = v;
  });
  return (double)g_clk_khz[dev];
}

}  // namespace tw

extern "C" {

int tw_version(void) { return TW_ABI_VERSION; }

const char* tw_last_error(void) { return g_last_error.c_str(); }

}  // extern "C"
