"""CPU tests of libbf16x_hip.so: exports, the host encoder, the plan builder
and argument validation of the GPU entry points (rejected before any launch)."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest
import torch

from oracle import dict_codec as dc
from tests.conftest import ROOT, golden_dict_cases

import bfloat16x_amd as bx
from bfloat16x_amd import _lib

HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def header_functions():
    names = set()
    for h in HEADERS:
        src = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(bf16x_[a-z0-9_]+)\s*\(", src))
    return sorted(names)


def test_library_exports_every_header_function():
    lib = _lib.lib()
    assert len(HEADERS) == 2
    names = header_functions()
    assert len(names) >= 23
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.PROTOTYPES, f"{n} has no ctypes prototype"
    assert bx.version().startswith("bf16x-hip")


def test_status_strings():
    assert _lib.status_string(0) == "ok"
    assert "sub" in _lib.status_string(_lib.ESUB)


@pytest.mark.parametrize("n", [1, 5, 31, 32, 33, 100, 4096, 4097])
def test_stream_words_matches_oracle(n):
    for b in (1, 3, 7):
        assert bx.stream_words(n, b) == dc.stream_words(n, b)


def _as_np(t):
    return t.numpy() if isinstance(t, torch.Tensor) else t


def test_encoder_matches_reference_golden(golden):
    for key, bits, sub in golden_dict_cases(golden):
        w = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
        d = bx.bf16x_quantize(w, sub=sub)
        for f in dc.__dict__.get("FIELDS", ()) or ("emax", "sign_packed", "mant_packed", "delta_packed",
                                                     "delta_ovf_idx", "delta_ovf_val"):
            ref = golden[key + "_" + f]
            got = _as_np(d[f])
            assert got.dtype == ref.dtype and np.array_equal(got, ref), (key, f)
        assert (d["out_f"], d["in_f"], d["sub"]) == (bits.shape[0], bits.shape[1], sub)


@pytest.mark.parametrize("shape,threads", [((64, 128), 1), ((33, 96), 3), ((128, 1536), 0), ((7, 9), 4)])
def test_encoder_matches_oracle(shape, threads):
    bits = dc.bench_weight_bits(*shape, seed=11)
    ref = dc.quantize(bits)
    w = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    d = bx.bf16x_quantize(w, n_threads=threads)
    for f in ("emax", "sign_packed", "mant_packed", "delta_packed", "delta_ovf_idx", "delta_ovf_val"):
        assert np.array_equal(_as_np(d[f]), ref[f]), f


def test_encoder_rounds_fp32_like_torch():
    w = torch.randn(16, 64) * 0.3
    d = bx.bf16x_quantize(w)
    bits = w.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    ref = dc.quantize(bits)
    assert np.array_equal(d["mant_packed"].numpy(), ref["mant_packed"])


def _apply_plan(d, plan):
    """Patch the oracle's saturated decode with a host plan."""
    out = dc.decode_saturated(d).reshape(-1).copy()
    off = plan.tile_off.numpy().view(np.uint32)
    ent = plan.tile_ent.numpy().view(np.uint32)[:plan.n_fix]
    in_f = d["in_f"]
    tpr = (in_f + 65535) // 65536
    for t in range(off.size - 1):
        row, seg = divmod(t, tpr)
        for e in range(off[t], off[t + 1]):
            out[row * in_f + seg * 65536 + (ent[e] >> 16)] = ent[e] & 0xFFFF
    return out.reshape(d["out_f"], in_f)


@pytest.mark.parametrize("shape", [(32, 96), (5, 2048), (3, 70000)])
def test_host_plan_makes_saturated_exact(shape):
    bits = dc.bench_weight_bits(*shape, seed=4)
    d = dc.quantize(bits)
    plan = bx.build_plan_host(d, check=2)
    pos, _ = dc.fix_table(d)
    assert plan.n_fix == pos.size
    assert np.array_equal(_apply_plan(d, plan), bits)


def test_host_plan_rejects_malformed_tables():
    bits = dc.bench_weight_bits(8, 64, seed=1)
    d = dc.quantize(bits)
    bad = dict(d)
    bad["delta_ovf_idx"] = d["delta_ovf_idx"][::-1].copy()          # unsorted
    with pytest.raises(bx.Bf16xError) as ei:
        bx.build_plan_host(bad, check=1)
    assert ei.value.status == _lib.ETABLE
    bad = dict(d)
    bad["delta_ovf_val"] = d["delta_ovf_val"].copy()
    bad["delta_ovf_val"][0] = 3                                     # val < 7
    with pytest.raises(bx.Bf16xError):
        bx.build_plan_host(bad, check=1)
    bad = dict(d)                                                   # missing entry
    bad["delta_ovf_idx"] = d["delta_ovf_idx"][1:].copy()
    bad["delta_ovf_val"] = d["delta_ovf_val"][1:].copy()
    with pytest.raises(bx.Bf16xError):
        bx.build_plan_host(bad, check=2)
    bad = dict(d)
    bad["sign_packed"] = d["sign_packed"][:-1].copy()               # short stream
    with pytest.raises(bx.Bf16xError) as ei:
        bx.build_plan_host(bad, check=0)
    assert ei.value.status == _lib.ESTREAM_LEN
    bad = dict(d)
    bad["sub"] = 8
    with pytest.raises(bx.Bf16xError):
        bx.build_plan_host(bad)


def test_gpu_entry_points_validate_before_launch():
    """Invalid arguments are rejected on the host, before any device access,
    so these calls are safe without a GPU (the pointers are never touched)."""
    lib = _lib.lib()
    fake = ctypes.c_void_p(4096)
    n = 64 * 64
    ws, wm, wd, ne = dc.stream_words(n, 1), dc.stream_words(n, 7), dc.stream_words(n, 3), n // 16
    # sub != 16
    assert lib.bf16x_decode(fake, ws, fake, wm, fake, wd, fake, ne, None, None, 64, 64, 8, 1, fake, None) == _lib.ESUB
    # short mantissa stream
    assert lib.bf16x_decode(fake, ws, fake, wm - 1, fake, wd, fake, ne, None, None, 64, 64, 16, 1, fake,
                            None) == _lib.ESTREAM_LEN
    # exact mode without a plan
    assert lib.bf16x_decode(fake, ws, fake, wm, fake, wd, fake, ne, None, None, 64, 64, 16, 0, fake,
                            None) == _lib.EARG
    # null output
    assert lib.bf16x_decode(fake, ws, fake, wm, fake, wd, fake, ne, None, None, 64, 64, 16, 1, None,
                            None) == _lib.EARG
    # GEMV: bad dtype, in_f % 32
    assert lib.bf16x_gemv(fake, 7, fake, ws, fake, wm, fake, wd, fake, ne, None, None, None, 64, 64, 16, 1, fake,
                          None) == _lib.EDTYPE
    n2 = 64 * 48
    assert lib.bf16x_gemv(fake, 0, fake, dc.stream_words(n2, 1), fake, dc.stream_words(n2, 7), fake,
                          dc.stream_words(n2, 3), fake, n2 // 16, None, None, None, 64, 48, 16, 1, fake,
                          None) == _lib.ESHAPE
    assert lib.bf16x_gemv(fake, 0, fake, ws, fake, wm, fake, wd, fake, ne, None, None, None, 0, 64, 16, 1, fake,
                          None) == _lib.ESHAPE
    # row-streaming GEMM: M in 1..16, in_f 2048 or 4096, bf16 x, a row plan in exact mode
    n3 = 32 * 2048
    w3 = (dc.stream_words(n3, 1), dc.stream_words(n3, 7), dc.stream_words(n3, 3), n3 // 16)

    def rows(M=4, x_dtype=0, y_dtype=0, mode=1, plan=(None, None), in_f=2048, w=w3):
        return lib.bf16x_gemm_rows(fake, x_dtype, M, fake, w[0], fake, w[1], fake, w[2], fake, w[3], plan[0], plan[1],
                                   32, in_f, 16, mode, fake, y_dtype, None)
    assert rows(M=0) == _lib.ESHAPE and rows(M=17) == _lib.ESHAPE
    n4 = 32 * 1024
    assert rows(in_f=1024, w=(dc.stream_words(n4, 1), dc.stream_words(n4, 7), dc.stream_words(n4, 3),
                              n4 // 16)) == _lib.ESHAPE
    assert rows(x_dtype=2) == _lib.EDTYPE and rows(y_dtype=1) == _lib.EDTYPE
    assert rows(mode=0) == _lib.EARG                                   # exact mode without a plan
    assert rows(w=(w3[0], w3[1] - 1, w3[2], w3[3])) == _lib.ESTREAM_LEN
    # the layer launch (qkv projection + decode attention + o projection):
    # out_f must be the qkv rows of the heads, in_f in (2048, 4096], max_len
    # in (256, 768], sync large enough and not its own clear buffer
    H, KV, in_f = 32, 8, 4096
    out_f = (H + 2 * KV) * 128
    sb = lib.bf16x_layer_front_sync_bytes()
    assert sb >= 4 * 1025

    def words(of, inf):
        n_ = of * inf
        return (dc.stream_words(n_, 1), dc.stream_words(n_, 7), dc.stream_words(n_, 3), n_ // 16)

    def lf(of=out_f, inf=in_f, L=640, nh=H, sync_bytes=sb, mode=1, clear=None, o_out_f=0):
        w_ = words(of, inf)
        o = (None,) * 3 + (0,) + (None, 0) * 4 + (None,) * 3 + (0, None)
        if o_out_f:
            wo = words(o_out_f, inf)
            o = (fake, ctypes.c_void_p(8192), fake, 4096, fake, wo[0], fake, wo[1], fake, wo[2], fake, wo[3],
                 None, None, None, o_out_f, ctypes.c_void_p(12288))
        return lib.bf16x_layer_front_decode(fake, fake, 1e-5, fake, 16, fake, w_[0], fake, w_[1], fake, w_[2], fake,
                                            w_[3], None, None, None, of, inf, mode, fake, fake, fake, nh, KV, 128, L,
                                            0.088, fake, fake, fake, *o, fake, clear, sync_bytes, None)
    assert lf(of=out_f - 128) == _lib.ESHAPE
    assert lf(inf=2048) == _lib.ESHAPE and lf(inf=4128) == _lib.ESHAPE
    assert lf(L=256) == _lib.ESHAPE and lf(L=769) == _lib.ESHAPE
    assert lf(nh=36, of=(36 + 2 * KV) * 128) == _lib.ESHAPE          # heads not a multiple of 8
    assert lf(sync_bytes=sb - 4) == _lib.ECAPACITY
    assert lf(mode=0) == _lib.EARG                                     # exact mode without a plan
    assert lf(clear=fake) == _lib.EARG                                 # clearing its own counters
    # an o stage whose input is not the attention output (in_f != n_heads * 128)
    assert lf(o_out_f=4096, nh=16, of=(16 + 2 * KV) * 128) == _lib.ESHAPE


def test_wrappers_refuse_cpu_tensors():
    d = bx.bf16x_quantize(torch.randn(8, 64))
    with pytest.raises(ValueError):
        bx.bf16x_decode(d["sign_packed"], d["mant_packed"], d["delta_packed"], d["emax"], 8, 64)
