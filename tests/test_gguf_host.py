"""CPU tests of the GGUF half-block host codec in libbf16x_hip.so (C++):
byte-identical to the oracle and to the reference's golden vectors, and the
argument validation of the GGUF device entry points (no launch)."""
import ctypes

import numpy as np
import pytest

from oracle import gguf_codec as gc

import bfloat16x_amd as bx
from bfloat16x_amd import _lib


def _specials():
    u = np.array([0x00000000, 0x80000000, 0x00000001, 0x807FFFFF, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001,
                  0x7F800001, 0xFFFFFFFF, 0x7F7FFFFF, 0x7F7F8000, 0x3F808000, 0x3F818000, 0x3F80FFFF, 0x00008000],
                 np.uint32)
    return u.view(np.float32)


def test_fp32_to_bf16_matches_oracle_and_golden(golden):
    rng = np.random.default_rng(3)
    x = np.concatenate([(rng.standard_normal(100000) * 50).astype(np.float32),
                        rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32),
                        _specials()])
    assert np.array_equal(bx.gguf.fp32_to_bf16_bits(x), gc.fp32_to_bf16_bits(x))
    assert np.array_equal(bx.gguf.fp32_to_bf16_bits(golden["gguf_x"]), golden["gguf_bf16_bits"])


def test_quantize_blocks_matches_golden(golden):
    blocks = bx.gguf.quantize_blocks(golden["gguf_x"])
    assert blocks.shape == golden["gguf_blocks"].shape and np.array_equal(blocks, golden["gguf_blocks"])
    rng0 = np.random.default_rng(0)                  # the reference self-test recipe (:203-207)
    w = (rng0.standard_normal((256, 512)) * 0.13).astype(np.float32)
    idx = rng0.choice(w.size, w.size // 200, replace=False)
    w.reshape(-1)[idx] *= rng0.standard_normal(len(idx)) * 8
    assert np.array_equal(bx.gguf.quantize_tensor(w)[:32], golden["gguf_selftest_blocks"])


@pytest.mark.parametrize("shape", [(1, 32), (3, 96), (64, 4096), (7, 1024)])
def test_quantize_blocks_matches_oracle(shape):
    w = gc.student_t_weights(*shape, seed=shape[0])
    w.reshape(-1)[:16] = _specials()
    assert np.array_equal(bx.gguf.quantize_blocks(w), gc.quantize_blocks(w))


def test_quantize_blocks_bf16_tensor_is_bitwise():
    import torch
    bits = np.random.default_rng(5).integers(0, 2**16, (8, 64), dtype=np.uint64).astype(np.uint16)
    t = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    assert np.array_equal(bx.gguf.quantize_blocks(t), gc.quantize_blocks_bits(bits).reshape(8, 2, 46))


def test_quantize_rejects_ragged():
    with pytest.raises(ValueError):
        bx.gguf.quantize_blocks(np.zeros((2, 33), np.float32))


def test_gguf_entry_points_validate_before_launch():
    lib = _lib.lib()
    fake = ctypes.c_void_p(4096)
    nb = 4 * 2
    n_bytes = nb * 46
    assert lib.bf16x_gguf_decode(fake, n_bytes, 4, 63, fake, 0, None) == _lib.ESHAPE        # in_f % 32
    assert lib.bf16x_gguf_decode(fake, n_bytes - 4, 4, 64, fake, 0, None) == _lib.ESTREAM_LEN
    assert lib.bf16x_gguf_decode(fake, n_bytes, 4, 64, fake, 7, None) == _lib.EDTYPE
    assert lib.bf16x_gguf_decode(None, n_bytes, 4, 64, fake, 0, None) == _lib.EARG
    assert lib.bf16x_gguf_gemv(fake, 2, fake, n_bytes, 4, 64, fake, 0, fake, 128, None) == _lib.EDTYPE  # fp32 x
    assert lib.bf16x_gguf_gemv(fake, 0, fake, n_bytes, 4, 64, fake, 0, fake, 64, None) == _lib.ECAPACITY
    assert lib.bf16x_gguf_gemv_workspace(4096) == 8192
