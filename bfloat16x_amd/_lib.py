"""ctypes binding of libbf16x_hip.so (the C ABI declared in include/bf16x_hip.h and
include/bf16x_llama.h).

torch is imported first on purpose: torch ships its own HIP runtime
(torch/lib/libamdhip64.so, soname libamdhip64.so.7).  Loading this library
after it makes the dynamic linker resolve our libamdhip64.so.7 dependency to
that same runtime, so torch's streams and device pointers are valid here.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbf16x_hip.so")

OK = 0
EARG, ESHAPE, ESTREAM_LEN, ETABLE, ECAPACITY, ESUB, EDTYPE = -1, -2, -3, -4, -5, -6, -7
BF16, F16, F32 = 0, 1, 2
EXACT, SATURATED = 0, 1

_c_i32, _c_i64, _c_u32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32
_P = ctypes.c_void_p

# name -> (restype, argtypes); every function of include/bf16x_hip.h and include/bf16x_llama.h
PROTOTYPES = {
    "bf16x_version": (ctypes.c_char_p, []),
    "bf16x_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "bf16x_stream_words": (_c_i64, [_c_i64, _c_i32]),
    "bf16x_plan_tiles": (_c_i64, [_c_i64, _c_i64]),
    "bf16x_encode_host": (ctypes.c_int, [_P, _c_i64, _c_i64, _c_i32, _P, _P, _P, _P, _P, _P, _c_i64,
                                         ctypes.POINTER(_c_i64), _c_i32]),
    "bf16x_encode_workspace": (_c_i64, [_c_i64, _c_i64]),
    "bf16x_encode": (ctypes.c_int, [_P, _c_i64, _c_i64, _c_i32, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P,
                                    _P, _c_i64, _P, _P, _c_i64, _P]),
    "bf16x_plan_host": (ctypes.c_int, [_P, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64,
                                       _c_i64, _c_i64, _c_i32, _P, _P, _P, _c_i64, ctypes.POINTER(_c_i64)]),
    "bf16x_plan_from_csr": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _c_i64, _c_i64, _c_i64, _P, _P, _P]),
    "bf16x_decode": (ctypes.c_int, [_P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _P,
                                    _c_i64, _c_i64, _c_i32, _c_i32, _P, _P]),
    "bf16x_gemv": (ctypes.c_int, [_P, _c_i32, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _P, _P,
                                  _c_i64, _c_i64, _c_i32, _c_i32, _P, _P]),
    "bf16x_kplan_size": (_c_i64, [_c_i64, _c_i64]),
    "bf16x_kplan_build": (ctypes.c_int, [_P, _P, _c_i64, _c_i64, _P, _P, _P]),
    "bf16x_gemm_workspace": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "bf16x_gemm": (ctypes.c_int, [_P, _c_i32, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _P,
                                  _c_i64, _c_i64, _c_i32, _c_i32, _P, _c_i32, _P, _c_i64, _P]),
    "bf16x_gemm_rows": (ctypes.c_int, [_P, _c_i32, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P,
                                       _P, _c_i64, _c_i64, _c_i32, _c_i32, _P, _c_i32, _P]),
    "bf16x_cplan_size": (_c_i64, [_c_i64, _c_i64]),
    "bf16x_cplan_build": (ctypes.c_int, [_P, _P, _c_i64, _c_i64, _P, _P, _P]),
    "bf16x_gemm_chunks": (ctypes.c_int, [_P, _c_i32, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P,
                                         _P, _c_i64, _c_i64, _c_i32, _c_i32, _P, _c_i32, _P]),
    "bf16x_fp32_to_bf16_host": (ctypes.c_int, [_P, _c_i64, _P, _c_i32]),
    "bf16x_gguf_quantize_host": (ctypes.c_int, [_P, _c_i64, _P, _c_i32]),
    "bf16x_gguf_decode": (ctypes.c_int, [_P, _c_i64, _c_i64, _c_i64, _P, _c_i32, _P]),
    "bf16x_gguf_gemv_workspace": (_c_i64, [_c_i64]),
    "bf16x_gguf_gemv": (ctypes.c_int, [_P, _c_i32, _P, _c_i64, _c_i64, _c_i64, _P, _c_i32, _P, _c_i64, _P]),
    "bf16x_gguf_gemv_noalloc": (ctypes.c_int, [_P, _c_i32, _P, _c_i64, _c_i64, _c_i64, _P, _c_i32, _P]),
    "bf16x_gguf_ovf_pack_host": (ctypes.c_int, [_P, _c_i64, _c_i64, _P, _P, _c_i64, ctypes.POINTER(_c_i64), _c_i32]),
    "bf16x_gguf_ovf_check_host": (ctypes.c_int, [_P, _c_i64, _c_i64, _c_i64, _P, _P, _c_i64]),
    "bf16x_gguf_decode_lossless": (ctypes.c_int, [_P, _c_i64, _c_i64, _c_i64, _P, _P, _c_i64, _P, _c_i32, _P]),
    "bf16x_gguf_gemv_lossless": (ctypes.c_int, [_P, _c_i32, _P, _c_i64, _c_i64, _c_i64, _P, _P, _c_i64, _P, _c_i32,
                                                _P, _c_i64, _P]),
    "bf16x_gguf_gemm_workspace": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "bf16x_gguf_gemm": (ctypes.c_int, [_P, _c_i32, _c_i64, _P, _c_i64, _P, _P, _c_i64, _c_i64, _P, _c_i32, _P,
                                       _c_i64, _P]),
    "bf16x_gguf_kplan_build": (ctypes.c_int, [_P, _P, _c_i64, _c_i64, _P, _P, _P]),
    # include/bf16x_llama.h
    "bf16x_rmsnorm": (ctypes.c_int, [_P, _P, _c_i64, _P, _P, _P, _c_i64, _c_i64, ctypes.c_float, _c_i32, _P]),
    "bf16x_rope_kv": (ctypes.c_int, [_P, _c_i64, _P, _P, _c_i64, _c_i64, _c_i64, _c_i64, _P, _P, _P, _P]),
    "bf16x_attention": (ctypes.c_int, [_P, _P, _P, _P, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float,
                                       _P, _P]),
    "bf16x_attention_decode_lds": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "bf16x_attention_decode_workspace": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "bf16x_attention_decode": (ctypes.c_int, [_P, _P, _P, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float, _P, _P,
                                              _P, _c_i64, _P, _P]),
    "bf16x_silu_mul": (ctypes.c_int, [_P, _c_i64, _c_i64, _c_i32, _P, _P]),
    "bf16x_gemv_norm": (ctypes.c_int, [_P, _P, _P, _P, ctypes.c_float, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P,
                                       _c_i64, _P, _P, _P, _c_i64, _c_i64, _c_i32, _c_i32, _P, _P]),
    "bf16x_gemv_swiglu": (ctypes.c_int, [_P, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _P, _P, _c_i64,
                                         _c_i64, _c_i32, _P, _P]),
    "bf16x_gemv_residual_slots": (_c_i64, [_c_i64, _c_i64]),
    "bf16x_gemv_residual": (ctypes.c_int, [_P, _P, _P, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64,
                                           _P, _P, _P, _c_i64, _c_i64, _c_i32, _P, _P]),
    "bf16x_gemv_prenormed": (ctypes.c_int, [_P, _P, ctypes.c_float, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64,
                                            _P, _c_i64, _P, _P, _P, _c_i64, _c_i64, _c_i32, _c_i32, _P, _P]),
    "bf16x_layer_front_sync_bytes": (_c_i64, []),
    "bf16x_layer_front_decode": (ctypes.c_int, [_P, _P, ctypes.c_float, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P,
                                                _c_i64, _P, _c_i64, _P, _P, _P, _c_i64, _c_i64, _c_i32, _P, _P, _P,
                                                _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float, _P, _P, _P,
                                                _P, _P, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64, _P, _c_i64,
                                                _P, _P, _P, _c_i64, _P, _P, _P, _c_i64, _P]),
    "bf16x_greedy_workspace_bytes": (_c_i64, []),
    "bf16x_greedy": (ctypes.c_int, [_P, _c_i64, _P, _P, _P, _c_i64, _P, _c_i64, _P]),
    # kernel-choice overrides (include/bf16x_hip.h)
    "bf16x_set_tuning": (ctypes.c_int, [_c_i32, _c_i64]),
    "bf16x_get_tuning": (_c_i64, [_c_i32]),
}

# keys of bf16x_set_tuning (BF16X_TUNE_* in include/bf16x_hip.h)
TUNE_KEYS = {
    "gemm_skinny2_max": 0, "gemm_skinny_max": 1, "gemm_bm": 2, "gemm_split": 3, "gemm_ws_min_rows": 4,
    "gemm_ws_split": 5, "skinny_waves": 6, "skinny2_kq": 7, "skinny2_split": 8, "gemv_iters": 9, "gemv_g": 10,
    "gemv_long": 11, "gemv_xm_slots": 12, "gguf_long": 13, "gguf_iters": 14, "attn_split": 15,
    "gemm_ws_grouped": 16, "gemm_ws_resident": 17, "attn_mfma": 18, "chunk_atoms": 19,
}

_LIB = None


class Bf16xError(RuntimeError):
    """A non-zero status returned by the C ABI."""

    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {status_string(status)} (status {status})")


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it was not built (there is no fallback)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m bfloat16x_amd.build` "
                               "(the BF16X engine has no CPU fallback)")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = h
    return _LIB


def status_string(status: int) -> str:
    try:
        return lib().bf16x_status_string(int(status)).decode()
    except Exception:  # pragma: no cover - only when the library itself is missing
        return "unknown"


def check(status: int, what: str) -> None:
    if status != OK:
        raise Bf16xError(int(status), what)


def ptr(t) -> int | None:
    """Data pointer of a tensor (None stays None)."""
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device):
    """Raw hipStream_t of torch's current stream on `device`."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def version() -> str:
    return lib().bf16x_version().decode()


class tuning:
    """Context manager over bf16x_set_tuning: forces kernel choices for the
    duration of a `with` block (a test and sweep hook), then restores the
    previous values.  tuning(gemm_ws_min_rows=1 << 30) keeps every GEMM off
    the wave-specialised kernel, for instance."""

    def __init__(self, **overrides: int):
        unknown = set(overrides) - set(TUNE_KEYS)
        if unknown:
            raise KeyError(f"unknown tuning keys {sorted(unknown)}")
        self.overrides = {TUNE_KEYS[k]: int(v) for k, v in overrides.items()}
        self.saved: dict[int, int] = {}

    def __enter__(self):
        L = lib()
        for k, v in self.overrides.items():
            self.saved[k] = int(L.bf16x_get_tuning(k))
            check(L.bf16x_set_tuning(k, v), "bf16x_set_tuning")
        return self

    def __exit__(self, *exc):
        L = lib()
        for k, v in self.saved.items():
            L.bf16x_set_tuning(k, v)
        return False
