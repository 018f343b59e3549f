#include "status.hpp"

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "redline_amd/rlk.h"

namespace rlk {
namespace {
thread_local char g_message[512] = "";
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_message, sizeof(g_message), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return RLK_OK;
  return fail(static_cast<int>(e), "%s: kernel launch failed: %s", what, hipGetErrorString(e));
}

int compute_units() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      v = 256;
    cus[dev] = v;  // the same value from any thread
  }
  return cus[dev];
}

int tune_knob(const char* name, int fallback) {
  const char* v = std::getenv(name);
  if (v == nullptr || *v == '\0') return fallback;
  return std::atoi(v);
}

}  // namespace rlk

extern "C" const char* rlk_last_error(void) { return rlk::g_message; }

extern "C" const char* rlk_version(void) { return "redline_amd 0.1.0 (gfx950)"; }
