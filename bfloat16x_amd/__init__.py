"""bfloat16x_amd -- MI355X (gfx950) engine for BF16X-compressed bf16 weights.

Call surface (mirrors the reference dfytensor/bfloat16x):
  bf16x_quantize                       opqk_linear.py:291
  bf16x_decode / bf16x_decode_triton   bf16x_triton_test.py:80
  bf16x_fused_gemv                     bf16x_fused.py:114
  bf16x_fused_gemm                     bf16x_gemm_fused.py:97
  gguf.quantize_blocks / dequantize_blocks / quantize_tensor / fp32_to_bf16_bits
                                       bf16x_gguf_block.py:44-93
  Bf16xFused, deploy_bf16x_fused       bf16x_fused.py:149-263
  Bf16xGemmLinear, deploy_bf16x_gemm   bf16x_gemm_fused.py:154-242
  BF16XLinear                          opqk_linear.py:327-407
  disk.pack_model_to_disk / replace_linears_from_packed / Bf16xStreamLinear
                                       pack_to_disk.py:40-265 (bf16x-v1 files)
  llama.LlamaStack / LlamaRunner       the caller harness (bench_fused_cpm5.py:27-57)
All GPU work runs in the HIP library libbf16x_hip.so through its C ABI
(include/bf16x_hip.h, include/bf16x_llama.h).
"""
from ._lib import Bf16xError, tuning, version
from .codec import Bf16xPlan, bf16x_quantize, build_plan_host, stream_words
from . import disk, gguf, llama
from .disk import Bf16xStreamLinear, pack_model_to_disk, replace_linears_from_packed
from .nn import BF16XLinear, Bf16xFused, Bf16xGemmLinear, deploy_bf16x_fused, deploy_bf16x_gemm
from .ops import (bf16x_decode, bf16x_decode_triton, bf16x_fused_gemm, bf16x_fused_gemv, bf16x_gemm,
                  bf16x_gemv)

__all__ = [
    "BF16XLinear", "Bf16xFused", "Bf16xGemmLinear", "deploy_bf16x_fused", "deploy_bf16x_gemm",
    "Bf16xError", "Bf16xPlan", "bf16x_decode", "bf16x_decode_triton", "bf16x_fused_gemm", "bf16x_fused_gemv",
    "bf16x_gemm", "bf16x_gemv",
    "bf16x_quantize", "build_plan_host", "gguf", "stream_words", "version",
    "disk", "llama", "Bf16xStreamLinear", "pack_model_to_disk", "replace_linears_from_packed", "tuning",
]
