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

int tune_knob(const char* name, int fallback) {
  const char* v = std::getenv(name);
  if (v == nullptr || *v == '\0') return fallback;
  return std::atoi(v);
}

}  // namespace rlk

extern "C" const char* rlk_last_error(void) { return rlk::g_message; }

extern "C" const char* rlk_version(void) { return "redline_amd 0.1.0 (gfx950)"; }
