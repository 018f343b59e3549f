// Host-side status reporting shared by the launchers: a per-thread error
// message behind rlk_last_error(), argument checks that fail before launch,
// and the post-launch hipGetLastError check.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdarg>

namespace rlk {

// Records a formatted message for rlk_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Status of the launch just issued: RLK_OK, or the hipError_t with a message
// naming `what`.
int launch_status(const char* what);

// Compute units of the current device (cached per device; 256 if the query
// fails).
int compute_units();

// Raises the dynamic-LDS limit of `kernel` on the current device to at least
// `bytes` (hipFuncSetAttribute), once per (device, kernel) and size: later
// calls are a lookup.
hipError_t grant_dynamic_lds(const void* kernel, size_t bytes);

// Launch-policy knobs: overrides for tuning experiments, read from the
// RLK_TUNE_* environment variables once per process and settable through
// rlk_set_tune_knob.
enum Knob {
  kGatherBs, kGatherNt, kNormTpr, kNormNt, kSwigluBs, kSwigluNt, kRopeWpt, kAttnPersist,
  kW4Cfg, kW8Cfg, kPrefillDma, kPrefillQs, kAttnPv, kRopeBiasTok, kNumKnobs
};

// The override of `knob`, or `fallback` when none is set.
int tune_knob(Knob knob, int fallback);

}  // namespace rlk
