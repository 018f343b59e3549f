// Kernel launch helper of the HIP sources: a plain triple-chevron launch, or,
// when rlk_time_next_launch armed a pair of events on this thread, a
// hipExtLaunchKernel whose start/stop events take the dispatch's own begin
// and end timestamps (the per-dispatch duration a profiler's kernel trace
// records), used by the benchmark to time single launches.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "status.hpp"

namespace rlk {

template <typename... P, typename... A>
inline void launch(void (*kernel)(P...), dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                   A... args) {
  const LaunchEvents ev = take_launch_events();
  if (ev.start != nullptr) {
    hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), stream, ev.start, ev.stop,
                          0u, static_cast<P>(args)...);
  } else {
    kernel<<<grid, block, lds, stream>>>(static_cast<P>(args)...);
  }
}

}  // namespace rlk
