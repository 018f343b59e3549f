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

// Environment override of a launch-policy knob (tuning experiments only);
// returns `fallback` when the variable is unset.
int tune_knob(const char* name, int fallback);

}  // namespace rlk
