"""Seeded random shapes through the packed-dict kernels, against the oracle.

Each case draws out_f, in_f, the row count, the activation dtype, exact
(with a row plan) or saturated, and, for the GEMM, the path.  Decode is held
bit for bit (special values planted); the GEMV and GEMM are held to the
north-star tolerance against a float64 product of the oracle's decoded weight
(max 1e-2 elementwise, floor 1e-3 of the output rms; median 2e-3 where a case
has 64 outputs or more: over fewer, the median is one output's bf16 rounding,
up to 2^-8).

fp32 activations enter the fused kernels as x = hi + lo, two bf16 halves, so
each term x_k w_k carries a relative error of at most 2^-16.  An output that
is the near-cancelling sum of large terms (|y| well below 1e-3 of the rms)
may then exceed the elementwise bound; such an output passes if its error is
within the dot product's own bound, 2^-15 sum_k |x_k w_k|.  The reference's
Triton GEMM takes fp32 activations through tl.dot in its default fp32 dot
precision (bf16x_gemm_fused.py:89-91)."""

import random

import numpy as np
import pytest
import torch

from oracle import dict_codec as dc
from tests.test_gpu_dict import bits_tensor, to_dev, with_specials

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


@pytest.fixture(scope="module")
def bx():
    import bfloat16x_amd as m
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return m


def _cases(seed, n, gemm):
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        in_f = rng.choice([32, 64, 96, 192, 512, 1536, 2048, 2048, 4096, 4096, 4160, 5376, 8192, 14336, 16416])
        out_f = rng.choice([1, 3, 7, 8, 16, 17, 31, 100, 257, 1000, 2061, 4100])
        m = rng.choice([1, 1, 2, 3, 5, 8, 11, 16, 16, 17, 33, 64, 65, 130, 256, 300]) if gemm else 1
        if out_f * in_f > 1 << 24 or m * out_f * in_f > 1 << 30:
            continue
        path = rng.choice(["auto", "fused"]) if gemm else "gemv"
        if path == "fused" and in_f % 64:
            path = "auto"
        out.append((out_f, in_f, m, rng.random() < 0.7, rng.choice(list(DTYPES)), path, rng.randrange(1 << 20)))
    return out


GEMM_CASES = _cases(7, 32, gemm=True)
GEMV_CASES = _cases(8, 24, gemm=False)


def _ids(cases):
    return [f"{o}x{i}-M{m}-{'exact' if ex else 'sat'}-{dt}-{p}" for o, i, m, ex, dt, p, _ in cases]


def _weight(bx, out_f, in_f, exact, seed):
    bits = dc.bench_weight_bits(out_f, in_f, seed=seed % 1000)
    bits[(bits & 0x7F80) >= 0x7000] = 0x3F80          # |w| >= 2^97 (and inf / nan) would overflow the output
    d = bx.bf16x_quantize(bits_tensor(bits))
    dn = {k: (v.numpy() if isinstance(v, torch.Tensor) else v) for k, v in d.items()}
    plan = bx.build_plan_host(d, device=DEV) if exact else None
    return to_dev(d), dn, plan


def _check(y, x, dn, exact, dtype_name):
    xd = x.double().numpy().reshape(-1, dn["in_f"])
    ref = dc.gemm_ref(dn, xd, saturated=not exact)
    yv = y.float().cpu().numpy().reshape(ref.shape).astype(np.float64)
    r = ref.reshape(-1)
    rms = float(np.sqrt(np.mean(r * r)))
    err = np.abs(yv - ref)
    e = err / np.maximum(np.abs(ref), 1e-3 * rms + 1e-30)
    ok = e <= 1e-2
    if dtype_name == "fp32":
        w = np.abs(dc.bits_to_f32(dc.decode_saturated(dn) if not exact else dc.decode_exact(dn)).astype(np.float64))
        bound = np.abs(xd) @ w.reshape(dn["out_f"], dn["in_f"]).T * 2.0 ** -15
        ok |= err <= bound
    assert ok.all(), f"max rel {e.max():.3e} at {int(np.argmax(e))} of {e.size} outputs"
    if e.size >= 64:
        assert np.median(e) <= 2e-3, f"median rel {np.median(e):.3e}"


@pytest.mark.parametrize("case", GEMV_CASES, ids=_ids(GEMV_CASES))
def test_random_decode_and_gemv(bx, case):
    out_f, in_f, _, exact, dt, _, seed = case
    print("random decode+gemv", out_f, in_f, exact, dt, seed, flush=True)
    # decode: special values planted, bit for bit against the oracle
    bits = with_specials(dc.bench_weight_bits(out_f, in_f, seed=seed % 1000), seed=seed % 997)
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    plan = bx.build_plan_host(d, device=DEV) if exact else None
    w = bx.bf16x_decode(g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f, plan=plan)
    got = w.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    dn = {k: (v.numpy() if isinstance(v, torch.Tensor) else v) for k, v in d.items()}
    want = bits if exact else dc.decode_saturated(dn).reshape(out_f, in_f)
    assert np.array_equal(got, want)
    # GEMV on a weight without values that overflow the product
    g, dn, plan = _weight(bx, out_f, in_f, exact, seed)
    x = torch.randn(in_f, generator=torch.Generator().manual_seed(seed)).to(DTYPES[dt])
    y = bx.bf16x_gemv(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                      plan=plan)
    assert y.shape == (out_f,)
    _check(y, x, dn, exact, dt)


@pytest.mark.parametrize("case", GEMM_CASES, ids=_ids(GEMM_CASES))
def test_random_gemm(bx, case):
    out_f, in_f, m, exact, dt, path, seed = case
    print("random gemm", out_f, in_f, m, exact, dt, path, seed, flush=True)
    g, dn, plan = _weight(bx, out_f, in_f, exact, seed)
    x = torch.randn(m, in_f, generator=torch.Generator().manual_seed(seed)).to(DTYPES[dt])
    y = bx.bf16x_gemm(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                      plan=plan, path=path)
    assert y.shape == (m, out_f) and y.dtype == x.dtype
    _check(y, x, dn, exact, dt)
