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

}  // namespace cascade
