// Host-side helpers shared by the libcascade_hip entry points.
#pragma once

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

}  // namespace cascade
