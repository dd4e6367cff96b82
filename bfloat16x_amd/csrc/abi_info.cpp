// Version and status strings of the C ABI.
#include "../../include/bf16x_hip.h"

extern "C" const char* bf16x_version(void) { return "bf16x-hip 0.1.0 gfx950"; }

extern "C" const char* bf16x_status_string(int status) {
  switch (status) {
    case BF16X_OK: return "ok";
    case BF16X_EARG: return "invalid argument (null pointer, misaligned pointer or bad enum)";
    case BF16X_ESHAPE: return "unsupported or inconsistent shape";
    case BF16X_ESTREAM_LEN: return "a packed stream is shorter than the shape requires";
    case BF16X_ETABLE: return "malformed overflow table";
    case BF16X_ECAPACITY: return "output capacity too small";
    case BF16X_ESUB: return "sub != 16 is not supported by the GPU kernels";
    case BF16X_EDTYPE: return "unsupported dtype code";
    default: return status > 0 ? "HIP runtime error" : "unknown status";
  }
}
