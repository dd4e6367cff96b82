"""CPU oracle for the BF16X decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain numpy (and torch on the CPU for the timing
baseline), the algorithms of the reference repository's hot path so that the
HIP engine in ``bfloat16x_amd`` can be checked against them.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker: the product never routes through this
code, and the product fails loudly when its HIP library is missing.

Modules
-------
``dict_codec``  BF16X packed-dict encoder / exact and saturated decoders /
                fp32 GEMV and GEMM references (opqk_linear.py,
                bf16x_triton_test.py, bf16x_fused.py, bf16x_gemm_fused.py).
``gguf_codec``  46-byte GGUF half-block codec (bf16x_gguf_block.py:29-93).
``cpu_path``    the reference's CPU decode+matmul path (``BF16XLinear``,
                opqk_linear.py:360-404), used as the timed CPU baseline.

How each function is pinned (i.e. checked against something other than its
own formula) is recorded in its docstring and exercised in
``tests/test_oracle_*.py``.  Functions without such a check say
"parity unpinned".
"""
