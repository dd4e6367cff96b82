"""CPU tests of the Llama harness: configuration checks, the rotary table
against its closed form, and argument validation of the decoder-stack entry
points (rejected before any launch)."""
import ctypes
import math

import numpy as np
import pytest
import torch

from bfloat16x_amd import _lib, llama
from bfloat16x_amd.codec import stream_words


def test_config_defaults_are_the_benchmark_stack():
    c = llama.LlamaConfig()
    assert (c.n_layers, c.hidden, c.ffn, c.n_heads, c.n_kv_heads, c.head_dim, c.vocab) == \
        (32, 4096, 14336, 32, 8, 128, 128256)
    assert c.qkv_rows == 6144
    # 32 x (6144 + 4096 + 28672) x 4096 + 32 x 4096 x 14336 linear weights (about 6.98e9)
    assert c.linear_params() == 32 * (6144 * 4096 + 4096 * 4096 + 28672 * 4096 + 4096 * 14336) == 6_979_321_856


@pytest.mark.parametrize("kw", [dict(head_dim=64, hidden=2048), dict(n_kv_heads=5), dict(hidden=4000),
                                dict(vocab=1001)])
def test_config_rejects_unsupported(kw):
    with pytest.raises(ValueError):
        llama.LlamaConfig(**kw)


def test_rope_table_closed_form():
    t = llama.rope_table(40, 5e5, "cpu").double().numpy()
    assert t.shape == (40, 64, 2)
    for p in (0, 1, 17, 39):
        for i in (0, 1, 31, 63):
            ang = p * 5e5 ** (-2 * i / 128)
            assert abs(t[p, i, 0] - math.cos(ang)) < 1e-5 and abs(t[p, i, 1] - math.sin(ang)) < 1e-5
    assert np.all(t[0, :, 0] == 1) and np.all(t[0, :, 1] == 0)


def _call(name, *args):
    return getattr(_lib.lib(), name)(*args)


def test_entry_points_validate_before_launch():
    # every call below is rejected by the host-side checks, so the pointers
    # are never dereferenced; `p` is a 16-byte aligned host address
    keep = ctypes.create_string_buffer(1 << 16)
    p = ctypes.addressof(keep) + (-ctypes.addressof(keep)) % 16
    # bad flags, bad n, misalignment, residual missing
    assert _call("bf16x_rmsnorm", p, None, 0, None, p, p, 1, 64, 1e-5, 4, None) == _lib.EARG
    assert _call("bf16x_rmsnorm", p, None, 0, None, p, p, 1, 60, 1e-5, 0, None) == _lib.ESHAPE
    assert _call("bf16x_rmsnorm", p, None, 0, None, p, p, 1, 8200, 1e-5, 0, None) == _lib.ESHAPE
    assert _call("bf16x_rmsnorm", p + 2, None, 0, None, p, p, 1, 64, 1e-5, 0, None) == _lib.EARG
    assert _call("bf16x_rmsnorm", p, None, 0, None, p, p, 1, 64, 1e-5, 1, None) == _lib.EARG
    assert _call("bf16x_rmsnorm", p, p, 0, p, p, p, 1, 64, 1e-5, 2, None) == _lib.EARG      # x_rows 0
    # rope: head_dim, head ratio
    assert _call("bf16x_rope_kv", p, 1, p, p, 32, 8, 64, 16, p, p, p, None) == _lib.ESHAPE
    assert _call("bf16x_rope_kv", p, 1, p, p, 30, 8, 128, 16, p, p, p, None) == _lib.ESHAPE
    assert _call("bf16x_rope_kv", None, 1, p, p, 32, 8, 128, 16, p, p, p, None) == _lib.EARG
    # attention: max_len above the LDS bound
    assert _call("bf16x_attention", p, p, p, p, 1, 32, 8, 128, 16385, 0.1, p, None) == _lib.ESHAPE
    assert _call("bf16x_attention", p, p + 4, p, p, 1, 32, 8, 128, 16, 0.1, p, None) == _lib.EARG
    # decode attention: unsupported head ratio, workspace too small
    assert _call("bf16x_attention_decode_lds", 24, 8, 640) == -1
    assert _call("bf16x_attention_decode_workspace", 32, 8, 640) > 0
    # every cache length the three decode kernels serve (one workgroup per kv
    # head, per query head, split) has a workspace size and a workgroup-memory size
    for L in (1, 256, 257, 768, 769, 4096, 16384):
        assert _call("bf16x_attention_decode_lds", 32, 8, L) > 0
        assert _call("bf16x_attention_decode_workspace", 32, 8, L) > 0
    assert _call("bf16x_attention_decode", p, p, p, 24, 8, 128, 640, 0.1, p, p, p, 1 << 20, p, None) == _lib.ESHAPE
    assert _call("bf16x_attention_decode", p, p, p, 32, 8, 128, 640, 0.1, p, p, p, 64, p, None) == _lib.ECAPACITY
    # silu_mul: ffn % 8, layout code
    assert _call("bf16x_silu_mul", p, 1, 12, 0, p, None) == _lib.ESHAPE
    assert _call("bf16x_silu_mul", p, 1, 16, 2, p, None) == _lib.EARG
    # SwiGLU GEMV: out_f % 8, in_f beyond one wave per row, mode
    def lens(o, i):
        n = o * i
        return stream_words(n, 1), stream_words(n, 7), stream_words(n, 3), (n + 15) // 16

    ls_, lm_, ld_, le_ = lens(12, 2048)
    assert _call("bf16x_gemv_swiglu", p, p, ls_, p, lm_, p, ld_, p, le_, p, p, p, 12, 2048, 1, p, None) == \
        _lib.ESHAPE                                                       # out_f % 8
    ls_, lm_, ld_, le_ = lens(16, 8192)
    assert _call("bf16x_gemv_swiglu", p, p, ls_, p, lm_, p, ld_, p, le_, p, p, p, 16, 8192, 1, p, None) == \
        _lib.ESHAPE                                                       # in_f > 4096
    ls_, lm_, ld_, le_ = lens(16, 128)
    assert _call("bf16x_gemv_swiglu", p, p, ls_, p, lm_, p, ld_, p, le_, p, p, p, 16, 128, 5, p, None) == _lib.EARG
    # norm GEMV: missing norm weight, bad epilogue, residual_out aliasing residual_in or x
    q = p + 4096
    norm_args = lambda x, ri, w, ro, epi: (x, ri, w, ro, 1e-5, p, ls_, p, lm_, p, ld_, p, le_, p, p, p, 16, 128, 1,
                                            epi, p, None)
    assert _call("bf16x_gemv_norm", *norm_args(p, q, None, p + 8192, 0)) == _lib.EARG
    assert _call("bf16x_gemv_norm", *norm_args(p, q, q, p + 8192, 2)) == _lib.EARG
    assert _call("bf16x_gemv_norm", *norm_args(p, q, q, q, 0)) == _lib.EARG
    assert _call("bf16x_gemv_norm", *norm_args(p, q, q, p, 0)) == _lib.EARG
    # greedy: misaligned token, history without length
    gw = int(_lib.lib().bf16x_greedy_workspace_bytes())
    assert _call("bf16x_greedy", p, 8, p + 4, p, p, 1, p, gw, None) == _lib.EARG
    assert _call("bf16x_greedy", p, 8, p, p, None, 1, p, gw, None) == _lib.EARG
    assert _call("bf16x_greedy", p, 0, p, p, p, 1, p, gw, None) == _lib.ESHAPE
    # workspace: missing, too small, misaligned
    assert _call("bf16x_greedy", p, 8, p, p, p, 1, None, gw, None) == _lib.EARG
    assert _call("bf16x_greedy", p, 8, p, p, p, 1, p, gw - 1, None) == _lib.ECAPACITY
    assert _call("bf16x_greedy", p, 8, p, p, p, 1, p + 4, gw, None) == _lib.EARG
    # a vocabulary whose last index batch would overflow the kernel's int indices
    assert _call("bf16x_greedy", p, 2 ** 31 - 1 - 2 * 1024 * 8 * 16 + 1, p, p, p, 1, p, gw, None) == _lib.ESHAPE
    # zero rows / tokens: nothing to launch
    assert _call("bf16x_rmsnorm", p, None, 0, None, p, p, 0, 64, 1e-5, 0, None) == _lib.OK
    assert _call("bf16x_silu_mul", p, 0, 16, 1, p, None) == _lib.OK


def test_wrappers_refuse_cpu_tensors():
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        llama.rmsnorm(x, torch.ones(64, dtype=torch.bfloat16), torch.empty_like(x))
    with pytest.raises(ValueError):
        llama.silu_mul(torch.zeros(2, 32, dtype=torch.bfloat16), torch.zeros(2, 16, dtype=torch.bfloat16), 16)
    with pytest.raises(RuntimeError):
        llama.LlamaStack(llama.LlamaConfig(n_layers=1, hidden=512, ffn=1024, n_heads=4, n_kv_heads=2, vocab=64))


def test_pairs8_rows_is_the_grouped_permutation():
    perm = llama.pairs8_rows(16)
    assert perm.tolist() == [0, 1, 2, 3, 16, 17, 18, 19, 4, 5, 6, 7, 20, 21, 22, 23,
                             8, 9, 10, 11, 24, 25, 26, 27, 12, 13, 14, 15, 28, 29, 30, 31]
    big = llama.pairs8_rows(14336)
    assert torch.equal(torch.sort(big).values, torch.arange(2 * 14336))


@pytest.mark.parametrize("n", [2, 3, 4, 5, 31, 32, 79])
def test_layer_front_buffers_alternate_cyclically(n):
    """Each layer launch clears the counters of the launch before it, so no
    two cyclically consecutive launches of a decode step (the graph repeats
    it) may share a buffer; three buffers suffice for any count."""
    c = llama.layer_front_buffers(n)
    assert len(c) == n and set(c) <= {0, 1, 2}
    assert all(c[k] != c[k - 1] for k in range(n))


def test_layer_front_buffers_need_two_launches():
    with pytest.raises(ValueError):
        llama.layer_front_buffers(1)
