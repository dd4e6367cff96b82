"""GPU parity of the row-streaming few-row fused decode+GEMM (bf16x_gemm_rows
in the C ABI: M <= 16, in_f 2048 or 4096; the bf16x_gemm_fused.py:97
contract at its smallest block) against the oracle.

fp32 activations that are exactly bf16 give y = the fp32 accumulation of one
pass, held to 1e-3 of the float64 product (a dropped or misplaced term, about
1/sqrt(in_f) of an output, fails it).  Rows of I pick W columns bit for bit,
which pins the LDS tile layout, the MFMA operand and result layouts and
every overflow patch, the dense patch loop included."""

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


def _np(d):
    return {k: (v.numpy() if isinstance(v, torch.Tensor) else v) for k, v in d.items()}


def _weight(bx, out_f, in_f, seed, specials=True):
    bits = dc.bench_weight_bits(out_f, in_f, seed=seed)
    if specials:
        bits = with_specials(bits, seed=seed + 1)
    bits[(bits & 0x7F00) == 0x7F00] = 0x3F80            # finite products
    d = bx.bf16x_quantize(bits_tensor(bits))
    return bits, d, to_dev(d), bx.build_plan_host(d, device=DEV)


def _rows(bx, x, g, out_f, in_f, plan, y_dtype=None):
    """bf16x_gemm_rows through the C ABI: y[M, out_f] in bf16 or fp32."""
    L = bx._lib.lib()
    yd = bx._lib.BF16 if y_dtype is None else y_dtype
    y = torch.empty(x.shape[0], out_f, dtype=torch.bfloat16 if yd == bx._lib.BF16 else torch.float32, device=DEV)
    st = L.bf16x_gemm_rows(x.data_ptr(), bx._lib.BF16, x.shape[0], g["sign_packed"].data_ptr(),
                           g["sign_packed"].numel(), g["mant_packed"].data_ptr(), g["mant_packed"].numel(),
                           g["delta_packed"].data_ptr(), g["delta_packed"].numel(), g["emax"].data_ptr(),
                           g["emax"].numel(), bx._lib.ptr(plan.tile_off) if plan is not None else None,
                           bx._lib.ptr(plan.tile_ent) if plan is not None else None, out_f, in_f, 16,
                           bx._lib.EXACT if plan is not None else bx._lib.SATURATED, y.data_ptr(), yd,
                           bx._lib.stream_of(x.device))
    bx._lib.check(st, "bf16x_gemm_rows")
    return y


# (M, out_f, in_f): every token count class (1, < 8, 8, > 8, 16), out_f below
# one 8-row group, ragged last groups, more groups than workgroups
CASES = [(1, 64, 2048), (2, 200, 4096), (5, 130, 4096), (8, 8, 2048), (9, 1000, 2048), (13, 2061, 4096),
         (16, 7, 4096), (16, 512, 2048), (16, 4100, 4096)]


@pytest.mark.parametrize("M,out_f,in_f", CASES)
def test_rows_fp32_product(bx, M, out_f, in_f):
    print("rows fp32", M, out_f, in_f, flush=True)
    bits, d, g, plan = _weight(bx, out_f, in_f, seed=M + out_f)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
    dn = _np(d)
    for p, sat in ((plan, False), (None, True)):
        y = _rows(bx, x.to(DEV), g, out_f, in_f, p, bx._lib.F32)
        assert y.shape == (M, out_f)
        mx, med = dc.rel_err(y.cpu().numpy(), dc.gemm_ref(dn, x.double().numpy(), saturated=sat))
        assert mx <= 1e-3 and med <= 1e-6, (sat, mx, med)
        yb = _rows(bx, x.to(DEV), g, out_f, in_f, p)
        check_tol(yb.float().cpu().numpy(), dc.gemm_ref(dn, x.float().numpy(), saturated=sat))


@pytest.mark.parametrize("M,out_f,in_f", [(3, 100, 4096), (16, 300, 2048)])
def test_rows_through_bf16x_gemm(bx, M, out_f, in_f):
    """bf16x_gemm (fused and auto) dispatches these shapes to the row kernel;
    fp32 activations are split into two bf16 passes (x = hi + lo)."""
    assert M <= bx.ops.GEMM_ROWS_MAX and in_f in bx.ops.GEMM_ROWS_IN_F
    bits, d, g, plan = _weight(bx, out_f, in_f, seed=M + 3)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(M + 3))
    for path in ("fused", "auto"):
        y = bx.bf16x_gemm(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                          plan=plan, path=path)
        assert y.dtype == torch.float32
        mx, med = dc.rel_err(y.cpu().numpy(), dc.gemm_ref(_np(d), x.double().numpy(), saturated=False))
        assert mx <= 1e-3 and med <= 1e-5, (path, mx, med)


@pytest.mark.parametrize("M,in_f", [(16, 2048), (11, 4096)])
def test_rows_identity_is_bit_exact(bx, M, in_f):
    out_f = 136
    bits, d, g, plan = _weight(bx, out_f, in_f, seed=M)
    bits = bits.copy()
    sat = dc.decode_saturated(_np(d))
    # the MFMA flushes subnormal inputs: compare those as zero
    for a in (bits, sat):
        a[(a & 0x7F80) == 0] = 0
    starts = list(range(0, in_f, M))
    if in_f == 4096:                     # every 4th window: each lane role and wave's K range still covered
        starts = starts[::4] + [starts[-1]]
    for start in starts:
        cols = min(M, in_f - start)
        eye = torch.zeros(M, in_f, dtype=torch.bfloat16)
        eye[torch.arange(cols), start + torch.arange(cols)] = 1
        for p, ref in ((plan, bits), (None, sat)):
            y = _rows(bx, eye.to(DEV), g, out_f, in_f, p)
            got = y.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)[:cols].T.copy()
            got[(got & 0x7F80) == 0] = 0
            assert np.array_equal(got, ref[:, start:start + cols]), (start, p is None)


def test_rows_dense_overflow(bx):
    """Rows with several hundred plan entries, past the 128 a wave preloads:
    the patch loop that reads the rest."""
    out_f, in_f, M = 40, 2048, 16
    rng = np.random.default_rng(9)
    bits = dc.bench_weight_bits(out_f, in_f, seed=9)
    tiny = rng.random(bits.shape) < 0.35
    bits[tiny] = (bits[tiny] & 0x807F) | 0x0080
    d = bx.bf16x_quantize(bits_tensor(bits))
    plan = bx.build_plan_host(d, device=DEV)
    assert plan.n_fix > out_f * 400
    g = to_dev(d)
    ref_bits = bits.copy()
    ref_bits[(ref_bits & 0x7F80) == 0] = 0
    for start in range(0, in_f, M):
        eye = torch.zeros(M, in_f, dtype=torch.bfloat16)
        eye[torch.arange(M), start + torch.arange(M)] = 1
        y = _rows(bx, eye.to(DEV), g, out_f, in_f, plan)
        got = y.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).T.copy()
        got[(got & 0x7F80) == 0] = 0
        assert np.array_equal(got, ref_bits[:, start:start + M]), start
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    y = _rows(bx, x.to(DEV), g, out_f, in_f, plan, bx._lib.F32)
    mx, med = dc.rel_err(y.cpu().numpy(), dc.gemm_ref(_np(d), x.double().numpy(), saturated=False))
    assert mx <= 1e-3 and med <= 1e-6, (mx, med)


def test_rows_rejects_other_shapes(bx):
    """M outside 1..16 and in_f other than 2048 / 4096 return BF16X_ESHAPE
    (streams long enough for the shape, so only the shape is wrong)."""
    out_f = 64
    L = bx._lib.lib()
    for M, in_f in ((17, 2048), (0, 2048), (4, 1024), (4, 14336)):
        _, _, g, _ = _weight(bx, out_f, in_f, seed=2, specials=False)
        x = torch.zeros(max(M, 1), in_f, dtype=torch.bfloat16, device=DEV)
        y = torch.empty(max(M, 1), out_f, dtype=torch.bfloat16, device=DEV)
        st = L.bf16x_gemm_rows(x.data_ptr(), bx._lib.BF16, M, g["sign_packed"].data_ptr(), g["sign_packed"].numel(),
                               g["mant_packed"].data_ptr(), g["mant_packed"].numel(), g["delta_packed"].data_ptr(),
                               g["delta_packed"].numel(), g["emax"].data_ptr(), g["emax"].numel(), None, None, out_f,
                               in_f, 16, bx._lib.SATURATED, y.data_ptr(), bx._lib.BF16, bx._lib.stream_of(x.device))
        assert st == bx._lib.ESHAPE, (M, in_f, st)


def test_rows_matches_skinny2(bx):
    """Same inputs through the 16x16x32 few-row kernel of bf16x_gemm (the
    row kernel switched off): both accumulate in fp32, so the fp32 outputs
    agree to accumulation-order rounding."""
    out_f, in_f, M = 520, 4096, 12
    bits, d, g, plan = _weight(bx, out_f, in_f, seed=6)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).float().to(DEV)
    y_rows = _rows(bx, x.to(torch.bfloat16), g, out_f, in_f, plan, bx._lib.F32).cpu().numpy()
    saved = bx.ops.GEMM_ROWS_MAX
    bx.ops.GEMM_ROWS_MAX = 0
    try:
        y_sk = bx.bf16x_gemm(x, g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                             plan=plan, path="fused").cpu().numpy()
    finally:
        bx.ops.GEMM_ROWS_MAX = saved
    scale = np.sqrt(np.mean(y_sk.astype(np.float64) ** 2))
    assert np.max(np.abs(y_rows.astype(np.float64) - y_sk)) <= 1e-5 * scale * np.sqrt(in_f)


@pytest.mark.parametrize("out_f,in_f", [(14336, 4096), (4096, 4096), (8192, 2048)])
@pytest.mark.parametrize("M", [1, 16])
def test_rows_full_size(bx, M, out_f, in_f):
    """Configuration-3 projection shapes (and a 2048-column weight), exact,
    against the fp32 product of the original weight on the device."""
    print("rows full", M, out_f, in_f, flush=True)
    bits = dc.bench_weight_bits(out_f, in_f, seed=1)
    w = bits_tensor(bits)
    d = bx.bf16x_quantize(w)
    g = to_dev(d)
    plan = bx.build_plan_host(d, device=DEV)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(DEV)
    y_ref = (x.float() @ w.to(DEV).float().t()).double().cpu().numpy()
    y = _rows(bx, x, g, out_f, in_f, plan)
    mx, med = check_tol(y.float().cpu().numpy(), y_ref)
    print("rows full-size rel err max %.2e median %.2e" % (mx, med), flush=True)


@pytest.mark.parametrize("lead", [(1,), (1, 1)])
def test_one_row_runs_the_gemv(bx, lead):
    """bf16x_gemm with one bf16 row returns the GEMV's output bit for bit (the
    dispatch sends it there), in the input's leading shape."""
    out_f, in_f = 1000, 4096
    bits, d, g, plan = _weight(bx, out_f, in_f, seed=31)
    x = torch.randn(*lead, in_f, generator=torch.Generator().manual_seed(31)).to(torch.bfloat16).to(DEV)
    for p in (plan, None):
        y = bx.bf16x_gemm(x, g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f, plan=p)
        yv = bx.bf16x_gemv(x.reshape(-1), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f,
                           in_f, plan=p)
        assert y.shape == (*lead, out_f) and y.dtype == torch.bfloat16
        assert torch.equal(y.reshape(-1).view(torch.int16), yv.view(torch.int16))
