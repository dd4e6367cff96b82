// Host-side helpers shared by the C-ABI launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/bf16x_hip.h"

// Kernel-choice override of bf16x_set_tuning (abi_info.cpp): -1 = automatic.
int64_t bf16x_tuning_value(int key);

namespace bf16x {
// Exclusive scan of a[0..n) in place on `st`, a[n] = the total (gemm.hip).
void scan_offsets(uint32_t* a, int64_t n, hipStream_t st);
}  // namespace bf16x

namespace {

inline int64_t tuning(int key) { return bf16x_tuning_value(key); }

inline bool aligned2(const void* p) { return ((uintptr_t)p & 1u) == 0; }
inline bool aligned4(const void* p) { return ((uintptr_t)p & 3u) == 0; }
inline bool aligned8(const void* p) { return ((uintptr_t)p & 7u) == 0; }
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Status of the launch just enqueued: 0 or the hipError_t (> 0).
inline int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BF16X_OK : (int)e;
}

constexpr int64_t kPlanTileCols = 65536;

// Shape / stream-length validation shared by every packed-dict entry point.
inline int check_dict(int64_t out_f, int64_t in_f, int32_t sub, int64_t n_sign, int64_t n_mant, int64_t n_delta,
                      int64_t n_emax) {
  if (out_f <= 0 || in_f <= 0) return BF16X_ESHAPE;
  if (sub != 16) return BF16X_ESUB;
  const int64_t N = out_f * in_f;
  if (N > ((int64_t)1 << 36)) return BF16X_ESHAPE;
  if (n_sign < bf16x_stream_words(N, 1) || n_mant < bf16x_stream_words(N, 7) ||
      n_delta < bf16x_stream_words(N, 3) || n_emax < (N + 15) / 16)
    return BF16X_ESTREAM_LEN;
  return BF16X_OK;
}

// Compute units of the current device (cached per device), or 0 when it
// cannot be queried.
inline int device_cus() {
  static int cache[64];
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] > 0) return cache[dev];
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 0;
  cache[dev] = cus;
  return cus;
}

inline int tiles_per_row(int64_t in_f) { return (int)((in_f + kPlanTileCols - 1) / kPlanTileCols); }

}  // namespace
