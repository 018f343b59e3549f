#include "status.hpp"

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <climits>
#include <mutex>

#include "redline_amd/rlk.h"

namespace rlk {
namespace {
thread_local char g_message[512] = "";
}  // namespace

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
  // One relaxed atomic per device: concurrent first launches may both query
  // the attribute, and both store the same value.
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

namespace {
struct LdsGrant {
  int dev;
  const void* kernel;
  size_t bytes;
};
std::mutex g_grant_mu;
LdsGrant g_grants[256];
int g_num_grants = 0;
}  // namespace

hipError_t grant_dynamic_lds(const void* kernel, size_t bytes) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_grant_mu);
  for (int i = 0; i < g_num_grants; ++i) {
    if (g_grants[i].dev == dev && g_grants[i].kernel == kernel && g_grants[i].bytes >= bytes)
      return hipSuccess;
  }
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(bytes));
  if (e != hipSuccess) return e;
  for (int i = 0; i < g_num_grants; ++i) {
    if (g_grants[i].dev == dev && g_grants[i].kernel == kernel) {
      g_grants[i].bytes = bytes;
      return hipSuccess;
    }
  }
  if (g_num_grants < 256) g_grants[g_num_grants++] = LdsGrant{dev, kernel, bytes};
  return hipSuccess;  // a full table only means the attribute is set again next time
}

namespace {
// Launch-policy overrides, indexed by Knob.  They are read from the
// environment once per process (the first launch) and can be changed only
// through rlk_set_tune_knob; a production launch therefore pays one atomic
// load per knob, and a variable inherited after start-up changes nothing.
constexpr const char* kKnobNames[kNumKnobs] = {
    "RLK_TUNE_GATHER_BS", "RLK_TUNE_GATHER_NT", "RLK_TUNE_NORM_TPR",   "RLK_TUNE_NORM_NT",
    "RLK_TUNE_SWIGLU_BS", "RLK_TUNE_SWIGLU_NT", "RLK_TUNE_ROPE_WPT",   "RLK_TUNE_ATTN_PERSIST",
    "RLK_TUNE_W4_CFG",    "RLK_TUNE_W8_CFG",    "RLK_TUNE_PREFILL_DMA", "RLK_TUNE_PREFILL_QS",
    "RLK_TUNE_ATTN_PV",   "RLK_TUNE_ROPE_BIAS_TOK",
};
constexpr int kUnset = INT_MIN;
std::atomic<int> g_knobs[kNumKnobs];
std::once_flag g_knobs_once;

void read_knobs_from_env() {
  for (int k = 0; k < kNumKnobs; ++k) {
    const char* v = std::getenv(kKnobNames[k]);
    g_knobs[k].store(v != nullptr && *v != '\0' ? std::atoi(v) : kUnset,
                     std::memory_order_relaxed);
  }
}
}  // namespace

int tune_knob(Knob knob, int fallback) {
  std::call_once(g_knobs_once, read_knobs_from_env);
  const int v = g_knobs[knob].load(std::memory_order_relaxed);
  return v == kUnset ? fallback : v;
}

}  // namespace rlk

extern "C" const char* rlk_last_error(void) { return rlk::g_message; }

extern "C" int rlk_set_tune_knob(const char* name, int value, int set) {
  std::call_once(rlk::g_knobs_once, rlk::read_knobs_from_env);
  if (name != nullptr) {
    for (int k = 0; k < rlk::kNumKnobs; ++k) {
      if (std::strcmp(name, rlk::kKnobNames[k]) == 0) {
        rlk::g_knobs[k].store(set ? value : rlk::kUnset, std::memory_order_relaxed);
        return RLK_OK;
      }
    }
  }
  return rlk::fail(RLK_EINVAL, "rlk_set_tune_knob: unknown knob '%s'", name ? name : "(null)");
}

extern "C" int rlk_get_tune_knob(const char* name, int* value, int* is_set) {
  std::call_once(rlk::g_knobs_once, rlk::read_knobs_from_env);
  if (name != nullptr && value != nullptr && is_set != nullptr) {
    for (int k = 0; k < rlk::kNumKnobs; ++k) {
      if (std::strcmp(name, rlk::kKnobNames[k]) == 0) {
        const int v = rlk::g_knobs[k].load(std::memory_order_relaxed);
        *is_set = v != rlk::kUnset;
        *value = *is_set ? v : 0;
        return RLK_OK;
      }
    }
  }
  return rlk::fail(RLK_EINVAL, "rlk_get_tune_knob: unknown knob '%s' or null output",
                   name ? name : "(null)");
}

extern "C" const char* rlk_version(void) { return "redline_amd 0.1.0 (gfx950)"; }
