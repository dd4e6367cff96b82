"""GPU parity of the few-row fused decode+GEMM (M <= 64, in_f % 128 == 0; the
16x16x32-MFMA kernel behind bf16x_gemm, bf16x_gemm_fused.py:97 contract)
against the oracle, through the C ABI.

Beside the bf16-output checks of test_gpu_gemm.py (which also reach this
kernel), the product is read in fp32 (fp32 activations that are exactly
bf16 give y = the fp32 accumulation of one pass) and held to 1e-3 of the
float64 product: a dropped or misplaced term (about 1/sqrt(in_f) of an
output) fails it.  Rows of I pick W columns bit for bit, which pins the
MFMA operand and result layouts and every overflow patch."""

import numpy as np
import pytest
import torch

from oracle import dict_codec as dc
from tests.test_gpu_dict import DEV, bits_tensor, check_tol, to_dev, with_specials

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def bx():
    import bfloat16x_amd as m
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return m


@pytest.fixture(autouse=True)
def _no_row_kernel(bx, monkeypatch):
    """bf16x_gemm runs the row-streaming kernel for M <= 16 at in_f 2048 /
    4096 (test_gpu_gemm_rows.py) and the GEMV for one bf16 row; these tests
    pin the 16x16x32 kernel."""
    monkeypatch.setattr(bx.ops, "GEMM_ROWS_MAX", 0)
    monkeypatch.setattr(bx.ops, "GEMM_ONE_ROW_GEMV", False)


def _np(d):
    return {k: (v.numpy() if isinstance(v, torch.Tensor) else v) for k, v in d.items()}


def _weight(bx, out_f, in_f, seed, specials=True):
    bits = dc.bench_weight_bits(out_f, in_f, seed=seed)
    if specials:
        bits = with_specials(bits, seed=seed + 1)
    bits[(bits & 0x7F00) == 0x7F00] = 0x3F80            # finite products
    d = bx.bf16x_quantize(bits_tensor(bits))
    return bits, d, to_dev(d), bx.build_plan_host(d, device=DEV)


def _gemm(bx, x, g, out_f, in_f, plan):
    return bx.bf16x_gemm(x, g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f, plan=plan,
                         path="fused")


# (M, out_f, in_f): one to four token blocks, ragged M and out_f (partial
# 64-row tiles and 32-row plan groups), K split or not
CASES = [(1, 64, 128), (2, 200, 1024), (5, 130, 4096), (16, 512, 1536), (17, 96, 2048), (31, 1000, 256),
         (32, 256, 4096), (33, 72, 1024), (48, 384, 14336), (64, 200, 2048)]


@pytest.mark.parametrize("M,out_f,in_f", CASES)
def test_skinny2_fp32_product(bx, M, out_f, in_f):
    print("skinny2 fp32", M, out_f, in_f, flush=True)
    bits, d, g, plan = _weight(bx, out_f, in_f, seed=M + out_f)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16).float()
    dn = _np(d)
    for p, sat in ((plan, False), (None, True)):
        y = _gemm(bx, x.to(DEV), g, out_f, in_f, p)
        assert y.dtype == torch.float32 and y.shape == (M, out_f)
        mx, med = dc.rel_err(y.cpu().numpy(), dc.gemm_ref(dn, x.double().numpy(), saturated=sat))
        assert mx <= 1e-3 and med <= 1e-6, (sat, mx, med)


@pytest.mark.parametrize("kq", ["1", "2"])
@pytest.mark.parametrize("M,out_f,in_f", [(5, 130, 4096), (33, 72, 1024), (48, 384, 14336), (64, 200, 2048)])
def test_skinny2_waves_per_row_group(bx, tune, kq, M, out_f, in_f):
    """The other wave-per-row-group counts (override skinny2_kq = 1: one wave
    walks every step of its rows; 2: two waves take alternate steps) give the
    same fp32 product: the default is 4 up to 32 rows and 2 above."""
    tune(skinny2_kq=int(kq))
    bits, d, g, plan = _weight(bx, out_f, in_f, seed=M + out_f + 7)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(M + 1)).to(torch.bfloat16).float()
    dn = _np(d)
    for p, sat in ((plan, False), (None, True)):
        y = _gemm(bx, x.to(DEV), g, out_f, in_f, p)
        mx, med = dc.rel_err(y.cpu().numpy(), dc.gemm_ref(dn, x.double().numpy(), saturated=sat))
        assert mx <= 1e-3 and med <= 1e-6, (kq, sat, mx, med)


@pytest.mark.parametrize("M", [1, 16, 40, 64])
def test_skinny2_identity_is_bit_exact(bx, M):
    out_f, in_f = 136, 512
    bits, d, g, plan = _weight(bx, out_f, in_f, seed=M)
    bits = bits.copy()
    sat = dc.decode_saturated(_np(d))
    # the MFMA flushes subnormal inputs: compare those as zero
    for a in (bits, sat):
        a[(a & 0x7F80) == 0] = 0
    for start in range(0, in_f, M):
        cols = min(M, in_f - start)
        eye = torch.zeros(M, in_f, dtype=torch.bfloat16)
        eye[torch.arange(cols), start + torch.arange(cols)] = 1
        for p, ref in ((plan, bits), (None, sat)):
            y = _gemm(bx, eye.to(DEV), g, out_f, in_f, p)
            got = y.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)[:cols].T.copy()
            got[(got & 0x7F80) == 0] = 0
            assert np.array_equal(got, ref[:, start:start + cols]), (start, p is None)


def test_skinny2_matches_previous_kernel(bx):
    """Same inputs through the 32x32-MFMA few-row kernel (selected by the
    override gemm_skinny2_max = 0): both accumulate in fp32, so the bf16
    outputs agree to within one rounding of either."""
    out_f, in_f, M = 320, 4096, 24
    bits, d, g, plan = _weight(bx, out_f, in_f, seed=4)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(DEV)
    y2 = _gemm(bx, x, g, out_f, in_f, plan).float().cpu().numpy()
    with bx.tuning(gemm_skinny2_max=0):
        y1 = _gemm(bx, x, g, out_f, in_f, plan).float().cpu().numpy()
    ref = dc.gemm_ref(_np(d), x.float().cpu().numpy(), saturated=False)
    check_tol(y2, ref)
    check_tol(y1, ref)
    ulp = np.abs(y1).astype(np.float64) * 2.0 ** -7 + 1e-6
    assert np.all(np.abs(y1.astype(np.float64) - y2) <= ulp + 1e-3 * np.sqrt(np.mean(ref * ref)))


def test_skinny2_dense_overflow(bx):
    """Runs longer than the 128 entries a lane pair preloads: the dense loop."""
    out_f, in_f, M = 96, 1024, 20
    rng = np.random.default_rng(9)
    bits = dc.bench_weight_bits(out_f, in_f, seed=9)
    tiny = rng.random(bits.shape) < 0.35
    bits[tiny] = (bits[tiny] & 0x807F) | 0x0080
    d = bx.bf16x_quantize(bits_tensor(bits))
    plan = bx.build_plan_host(d, device=DEV)
    assert plan.n_fix > out_f * in_f // 32 * 4
    g = to_dev(d)
    eye = torch.zeros(M, in_f, dtype=torch.bfloat16)
    for start in range(0, in_f, M):
        cols = min(M, in_f - start)
        eye.zero_()
        eye[torch.arange(cols), start + torch.arange(cols)] = 1
        y = _gemm(bx, eye.to(DEV), g, out_f, in_f, plan)
        got = y.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)[:cols].T.copy()
        ref = bits[:, start:start + cols].copy()
        for a in (got, ref):
            a[(a & 0x7F80) == 0] = 0
        assert np.array_equal(got, ref), start


@pytest.mark.parametrize("out_f,in_f", [(14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("M", [1, 16, 64])
def test_skinny2_full_size(bx, M, out_f, in_f):
    """Configuration-3 projection shapes, exact, against the fp32 product of
    the original weight on the device."""
    print("skinny2 full", M, out_f, in_f, flush=True)
    bits = dc.bench_weight_bits(out_f, in_f, seed=1)
    w = bits_tensor(bits)
    d = bx.bf16x_quantize(w)
    g = to_dev(d)
    plan = bx.build_plan_host(d, device=DEV)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(DEV)
    y_ref = (x.float() @ w.to(DEV).float().t()).double().cpu().numpy()
    y = _gemm(bx, x, g, out_f, in_f, plan)
    mx, med = check_tol(y.float().cpu().numpy(), y_ref)
    print("skinny2 full-size rel err max %.2e median %.2e" % (mx, med), flush=True)
    assert bx._lib.lib().bf16x_get_tuning(bx._lib.TUNE_KEYS["gemm_skinny2_max"]) == -1
