// Host-side helpers shared by the libcascade_hip entry points.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/cascade_hip.h"

namespace cascade {

// The GEMV kernels keep the whole input vector in LDS (2 bytes / element).
constexpr int64_t kMaxGemvLdsBytes = 64 * 1024;

inline bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// fp32 logits[r] = W[r] . h for r < rows (gemv.hip); K a multiple of 8,
// K * 2 <= kMaxGemvLdsBytes, pointers 16-byte aligned.
hipError_t launch_logits_gemv(const uint16_t *w, int64_t rows, int64_t k,
                              const uint16_t *h, float *logits,
                              hipStream_t stream);

// Events set by cascade_time_next_launch for the calling thread's next
// kernel launch; taking them clears them.
struct LaunchEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
LaunchEvents take_launch_events();

// Every kernel of the library is launched through here.  When events are
// pending, hipExtLaunchKernelGGL binds them to the kernel's own execution:
// their elapsed time is the kernel's duration, without the dispatch time a
// pair of stream markers around the launch would include.
template <typename Kernel, typename... Args>
hipError_t launch_kernel(Kernel kernel, dim3 grid, dim3 block, size_t lds,
                         hipStream_t s, Args... args) {
  const LaunchEvents ev = take_launch_events();
  if (ev.start != nullptr || ev.stop != nullptr)
    hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), s,
                          ev.start, ev.stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
  return hipGetLastError();
}

}  // namespace cascade
