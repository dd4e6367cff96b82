// Version and status strings of the C ABI, and the kernel-choice overrides.
#include <atomic>

#include "../../include/bf16x_hip.h"

extern "C" const char* bf16x_version(void) { return "bf16x-hip 0.1.0 gfx950"; }

extern "C" const char* bf16x_status_string(int status) {
  switch (status) {
    case BF16X_OK: return "ok";
    case BF16X_EARG: return "invalid argument (null pointer, misaligned pointer or bad enum)";
    case BF16X_ESHAPE: return "unsupported or inconsistent shape";
    case BF16X_ESTREAM_LEN: return "a packed stream is shorter than the shape requires";
    case BF16X_ETABLE: return "malformed overflow table";
    case BF16X_ECAPACITY:
      return "capacity too small (an output or workspace, or the fixed scratch of an allocation-free entry point)";
    case BF16X_ESUB: return "sub != 16 is not supported by the GPU kernels";
    case BF16X_EDTYPE: return "unsupported dtype code";
    default: return status > 0 ? "HIP runtime error" : "unknown status";
  }
}

// Overrides stored as value + 1 so the zero-initialised table means
// "automatic" for every key.
static std::atomic<int64_t> g_tuning[BF16X_TUNE_COUNT];

int64_t bf16x_tuning_value(int key) {
  if (key < 0 || key >= BF16X_TUNE_COUNT) return -1;
  return g_tuning[key].load(std::memory_order_relaxed) - 1;
}

extern "C" int bf16x_set_tuning(int32_t key, int64_t value) {
  if (key < 0 || key >= BF16X_TUNE_COUNT) return BF16X_EARG;
  g_tuning[key].store(value < 0 ? 0 : value + 1, std::memory_order_relaxed);
  return BF16X_OK;
}

extern "C" int64_t bf16x_get_tuning(int32_t key) { return bf16x_tuning_value(key); }
