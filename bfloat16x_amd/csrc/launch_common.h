// Host-side helpers shared by the C-ABI launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/bf16x_hip.h"

namespace {

inline bool aligned2(const void* p) { return ((uintptr_t)p & 1u) == 0; }
inline bool aligned4(const void* p) { return ((uintptr_t)p & 3u) == 0; }
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Status of the launch just enqueued: 0 or the hipError_t (> 0).
inline int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BF16X_OK : (int)e;
}

}  // namespace
