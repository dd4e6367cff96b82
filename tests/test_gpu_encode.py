"""GPU tests of the device encoder (bf16x_encode): the dict of a GPU weight
is byte-identical to the reference's golden dicts and to the host encoder,
for odd sizes (N not a multiple of 32, N < 32), special values (+-0,
denormals, inf, NaN, exponent 255), configuration 1 and the headline shape."""
import numpy as np
import pytest
import torch

from oracle import dict_codec as dc
from tests.conftest import golden_dict_cases
from tests.test_gpu_dict import DEV

pytestmark = pytest.mark.gpu

FIELDS = ("emax", "sign_packed", "mant_packed", "delta_packed", "delta_ovf_idx", "delta_ovf_val")


@pytest.fixture(scope="module")
def bx():
    import bfloat16x_amd as m
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return m


def same_dict(a, b, what):
    for f in FIELDS:
        x, y = a[f].cpu().numpy(), b[f].cpu().numpy()
        assert x.dtype == y.dtype and np.array_equal(x, y), (what, f, x.shape, y.shape)
    assert (a["out_f"], a["in_f"], a["sub"]) == (b["out_f"], b["in_f"], b["sub"])


def test_device_encoder_matches_reference_golden(bx, golden):
    n = 0
    for key, bits, sub in golden_dict_cases(golden):
        if sub != 16:
            continue
        w = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
        d = bx.bf16x_quantize(w)
        assert d["sign_packed"].is_cuda
        for f in FIELDS:
            ref = golden[key + "_" + f]
            got = d[f].cpu().numpy()
            assert got.dtype == ref.dtype and np.array_equal(got, ref), (key, f)
        n += 1
    assert n > 0


def special_bits(shape, seed):
    rng = np.random.default_rng(seed)
    e = rng.integers(100, 135, size=shape)
    b = ((rng.integers(0, 2, size=shape) << 15) | (e << 7) | rng.integers(0, 128, size=shape)).astype(np.uint16)
    flat = b.reshape(-1)
    k = flat.size
    flat[rng.choice(k, k // 20, replace=False)] = 0x0000                # +0
    flat[rng.choice(k, k // 20, replace=False)] = 0x8000                # -0
    flat[rng.choice(k, k // 20, replace=False)] = 0x0005                # denormals
    flat[rng.choice(k, k // 50, replace=False)] = 0x7F80                # +inf
    flat[rng.choice(k, k // 50, replace=False)] = 0xFFC1                # NaN
    flat[rng.choice(k, k // 50, replace=False)] = 0x7F00                # exponent 254
    return b


SHAPES = [(1, 1), (1, 31), (3, 7), (5, 33), (7, 9), (2, 48), (64, 4096), (33, 96), (300, 577)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("kind", ["bench", "special"])
def test_device_encoder_matches_host(bx, shape, kind):
    bits = dc.bench_weight_bits(*shape, seed=3) if kind == "bench" else special_bits(shape, 4)
    w = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
    same_dict(bx.bf16x_quantize(w.to(DEV)), bx.bf16x_quantize(w), (kind, shape))


@pytest.mark.parametrize("shape", [(2048, 1536), (14336, 4096)])
def test_device_encoder_config_shapes(bx, shape):
    bits = dc.bench_weight_bits(*shape, seed=0)
    w = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
    dd = bx.bf16x_quantize(w.to(DEV))
    same_dict(dd, bx.bf16x_quantize(w), shape)
    # and the device dict decodes back to the weight on the device
    plan = bx.build_plan_host(dd, device=DEV)
    dec = bx.bf16x_decode(dd["sign_packed"], dd["mant_packed"], dd["delta_packed"], dd["emax"], *shape, plan=plan)
    assert torch.equal(dec.view(torch.int16).cpu(), w.view(torch.int16))
