"""GPU parity of the fused decode+GEMM (bf16x_fused_gemm, bf16x_gemm_fused.py:97)
against the oracle: saturated (the reference kernel's numerics) and exact
(with the plan), through the C ABI."""
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


# (M, out_f, in_f): every tile configuration (M <= 32, <= 64, <= 128, > 128),
# ragged M and out_f, the C3 prefill shapes at reduced out_f
CASES = [(1, 128, 64), (5, 96, 128), (16, 512, 4096), (33, 200, 1536), (64, 1024, 4096), (100, 300, 1536),
         (128, 256, 14336), (256, 1024, 4096), (300, 130, 640), (512, 512, 4096), (2048, 256, 4096)]


@pytest.mark.parametrize("path", ["fused", "auto"])
@pytest.mark.parametrize("M,out_f,in_f", CASES)
def test_gemm_saturated_and_exact(bx, M, out_f, in_f, path):
    print("gemm", M, out_f, in_f, path, flush=True)
    bits = with_specials(dc.bench_weight_bits(out_f, in_f, seed=M), seed=3) if out_f * in_f < 1 << 20 else \
        dc.bench_weight_bits(out_f, in_f, seed=M)
    bits[(bits & 0x7F00) == 0x7F00] = 0x3F80        # no inf/nan/near-max: keep the products finite
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    dn = _np(d)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
    xn = x.float().numpy()
    y = bx.bf16x_fused_gemm(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                            path=path)
    assert y.dtype == torch.bfloat16 and y.shape == (M, out_f)
    check_tol(y.float().cpu().numpy(), dc.gemm_ref(dn, xn, saturated=True))
    plan = bx.build_plan_host(d, device=DEV)
    ye = bx.bf16x_fused_gemm(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                             plan=plan, path=path)
    check_tol(ye.float().cpu().numpy(), dc.gemm_ref(dn, xn, saturated=False))


def test_gemm_exact_dense_overflow(bx):
    """A weight with many overflow entries per row (every atom has several),
    so the plan window refills inside one atom."""
    out_f, in_f, M = 64, 1024, 48
    rng = np.random.default_rng(7)
    bits = dc.bench_weight_bits(out_f, in_f, seed=7)
    tiny = rng.random(bits.shape) < 0.3
    bits[tiny] = (bits[tiny] & 0x807F) | 0x0080              # exponent 1: delta >= 7 next to normal values
    d = bx.bf16x_quantize(bits_tensor(bits))
    plan = bx.build_plan_host(d, device=DEV)
    assert plan.n_fix > out_f * in_f // 32 * 2
    g = to_dev(d)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    y = bx.bf16x_gemm(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                      plan=plan, path="fused")
    # bit-level check of the weight the kernel used: x = unit rows picks W columns
    eye = torch.eye(in_f, dtype=torch.bfloat16)[:256]
    w_cols = bx.bf16x_gemm(eye.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                           plan=plan, path="fused")
    assert np.array_equal(w_cols.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).T, bits[:, :256])
    check_tol(y.float().cpu().numpy(), dc.gemm_ref(_np(d), x.float().numpy(), saturated=False))


def test_gemm_identity_is_bit_exact(bx):
    """x = I: the GEMM returns W^T element for element (one product per output,
    fp32 accumulate, bf16 store), so the decode inside the GEMM is bit exact."""
    out_f, in_f = 320, 512
    bits = dc.bench_weight_bits(out_f, in_f, seed=12)
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    plan = bx.build_plan_host(d, device=DEV)
    for start in range(0, in_f, 256):
        eye = torch.zeros(256, in_f, dtype=torch.bfloat16)
        eye[torch.arange(256), start + torch.arange(256)] = 1
        for p, ref in ((plan, bits), (None, dc.decode_saturated(_np(d)))):
            y = bx.bf16x_gemm(eye.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f,
                              in_f, plan=p, path="fused")
            got = y.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).T
            assert np.array_equal(got, ref[:, start:start + 256]), start


@pytest.mark.parametrize("xdt", [torch.float16, torch.float32])
def test_gemm_fp16_fp32_activations(bx, xdt):
    out_f, in_f, M = 256, 2048, 40
    bits = dc.bench_weight_bits(out_f, in_f, seed=5)
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    plan = bx.build_plan_host(d, device=DEV)
    x = torch.randn(2, M // 2, in_f, generator=torch.Generator().manual_seed(6)).to(xdt)
    y = bx.bf16x_gemm(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                      plan=plan, path="fused")
    assert y.dtype == xdt and y.shape == (2, M // 2, out_f)
    y_ref = dc.gemm_ref(_np(d), x.double().numpy().reshape(M, in_f), saturated=False)
    # fp16 splits exactly into two bf16; fp32 keeps 16 of its 24 mantissa bits
    # (max 1e-2 / median 2e-3, covers both)
    tol = dict(max_tol=2e-3, med_tol=5e-4) if xdt == torch.float16 else dict(max_tol=1e-2, med_tol=1e-5)
    check_tol(y.float().cpu().numpy().reshape(M, out_f), y_ref, **tol)


def test_gemm_unfused_shapes(bx):
    """in_f not a multiple of 64 (and > 65536) goes through decode + matmul."""
    for out_f, in_f, M in ((40, 96, 7), (3, 70016, 4)):
        bits = dc.bench_weight_bits(out_f, in_f, seed=in_f)
        d = bx.bf16x_quantize(bits_tensor(bits))
        g = to_dev(d)
        plan = bx.build_plan_host(d, device=DEV)
        x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
        y = bx.bf16x_gemm(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                          plan=plan)
        check_tol(y.float().cpu().numpy(), dc.gemm_ref(_np(d), x.float().numpy(), saturated=False))


def test_gemm_full_size(bx):
    """C3 shape 14336x4096 at M = 512, exact: against fp32 matmul of the
    original weight on the device."""
    out_f, in_f, M = 14336, 4096, 512
    print("gemm full", M, out_f, in_f, flush=True)
    bits = dc.bench_weight_bits(out_f, in_f, seed=0)
    w = bits_tensor(bits)
    d = bx.bf16x_quantize(w)
    g = to_dev(d)
    plan = bx.build_plan_host(d, device=DEV)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(DEV)
    y_ref = (x.float() @ w.to(DEV).float().t()).double().cpu().numpy()
    for path in ("fused", "auto"):
        y = bx.bf16x_gemm(x, g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f, plan=plan,
                          path=path)
        mx, med = check_tol(y.float().cpu().numpy(), y_ref)
        print("full-size gemm (%s) rel err max %.2e median %.2e" % (path, mx, med), flush=True)


@pytest.mark.parametrize("M", [32, 64, 100])
def test_gemm_few_rows_identity_is_bit_exact(bx, M):
    """The few-row kernel (M <= 128): x = rows of I select W columns, so the
    decode that feeds its MFMA is checked bit for bit, exact and saturated."""
    out_f, in_f = 96, 1024
    bits = with_specials(dc.bench_weight_bits(out_f, in_f, seed=M), seed=M)
    bits[(bits & 0x7F00) == 0x7F00] = 0x3F80
    bits[(bits & 0x7F80) == 0] = 0                       # MFMA inputs: no subnormals
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    plan = bx.build_plan_host(d, device=DEV)
    sat = dc.decode_saturated(_np(d))
    sat[(sat & 0x7F80) == 0] = 0
    for start in range(0, in_f, M):
        cols = min(M, in_f - start)
        eye = torch.zeros(M, in_f, dtype=torch.bfloat16)
        eye[torch.arange(cols), start + torch.arange(cols)] = 1
        for p, ref in ((plan, bits), (None, sat)):
            y = bx.bf16x_gemm(eye.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f,
                              in_f, plan=p, path="fused")
            got = y.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)[:cols].T
            assert np.array_equal(got, ref[:, start:start + cols]), (start, p is None)


# The wave-specialised kernel (M >= 192): four-step groups when in_f % 256 == 0
# (grouped = 1, the default there) and one-step tiles otherwise or when forced
# (grouped = 0); K splits forced to 1 and 3 (3 leaves a shorter last split).
@pytest.mark.parametrize("grouped", [1, 0])
@pytest.mark.parametrize("split", [-1, 1, 3])
@pytest.mark.parametrize("M,out_f,in_f", [(300, 300, 4096), (192, 136, 1024), (260, 256, 3072)])
def test_gemm_ws_groups_and_splits(bx, tune, grouped, split, M, out_f, in_f):
    print("gemm ws", M, out_f, in_f, "grouped", grouped, "split", split, flush=True)
    tune(gemm_ws_grouped=grouped, gemm_ws_split=split)
    bits = dc.bench_weight_bits(out_f, in_f, seed=out_f + split)
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    dn = _np(d)
    plan = bx.build_plan_host(d, device=DEV)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(M + split)).to(torch.bfloat16)
    for p, sat in ((plan, False), (None, True)):
        y = bx.bf16x_gemm(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                          plan=p, path="fused")
        check_tol(y.float().cpu().numpy(), dc.gemm_ref(dn, x.float().numpy(), saturated=sat))
    # the weight the kernel used, bit for bit: x = rows of I select W columns
    eye = torch.zeros(M, in_f, dtype=torch.bfloat16)
    cols = torch.arange(M) * (in_f // M)
    eye[torch.arange(M), cols] = 1
    w_cols = bx.bf16x_gemm(eye.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                           plan=plan, path="fused")
    got = w_cols.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    want = bits[:, cols.numpy()].T
    flush = (want & 0x7F80) == 0                # zeros and subnormals (the MFMA flushes these) come back as 0
    assert np.array_equal(np.where(flush, 0, got), np.where(flush, 0, want))
    assert not np.any(got[flush] & 0x7FFF)


# Whole-K tiles in full rounds, then the last round's tiles split over K: with
# the resident block count forced to 4 or 5, the 6 tiles of 300 x 300 run as
# 4 whole tiles + 2 tiles x 2 K ranges, or 5 whole tiles + 1 tile x 5 ranges
# (4 with four-step groups: 16 groups in ranges of 4); 520 rows x 200 columns
# (6 tiles, 3 M tiles) with 4 resident leaves the split tiles in two M rows.
@pytest.mark.parametrize("grouped", [1, 0])
@pytest.mark.parametrize("resident", [4, 5])
@pytest.mark.parametrize("M,out_f,in_f", [(300, 300, 4096), (520, 200, 1024)])
def test_gemm_ws_mixed_rounds(bx, tune, grouped, resident, M, out_f, in_f):
    print("gemm ws mixed", M, out_f, in_f, "grouped", grouped, "resident", resident, flush=True)
    tune(gemm_ws_grouped=grouped, gemm_ws_resident=resident)
    bits = dc.bench_weight_bits(out_f, in_f, seed=resident)
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    dn = _np(d)
    plan = bx.build_plan_host(d, device=DEV)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(M + resident)).to(torch.bfloat16)
    for p, sat in ((plan, False), (None, True)):
        for dt in (torch.bfloat16, torch.float32):
            y = bx.bf16x_gemm(x.to(DEV).to(dt), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"],
                              out_f, in_f, plan=p, path="fused")
            assert y.dtype == dt
            check_tol(y.float().cpu().numpy(), dc.gemm_ref(dn, x.float().numpy(), saturated=sat))


# Split tiles' fp32 partials are summed in K-range order by the reduction
# launch: repeated launches give the same bits, fp32 and bf16, and the
# result is the product to the north-star tolerance.
@pytest.mark.parametrize("split", [2, 5])
def test_gemm_ws_split_sum_is_deterministic(bx, tune, split):
    M, out_f, in_f = 256, 1024, 4096
    print("gemm ws split determinism", split, flush=True)
    tune(gemm_ws_split=split)
    bits = dc.bench_weight_bits(out_f, in_f, seed=split)
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    plan = bx.build_plan_host(d, device=DEV)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(split)).to(torch.bfloat16).to(DEV)
    for dt in (torch.float32, torch.bfloat16):
        xs = x.to(dt)
        ys = [bx.bf16x_gemm(xs, g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                            plan=plan, path="fused") for _ in range(4)]
        for yk in ys[1:]:
            assert torch.equal(yk.view(torch.int32 if dt == torch.float32 else torch.int16),
                               ys[0].view(torch.int32 if dt == torch.float32 else torch.int16))
    mx, med = dc.rel_err(ys[0].float().cpu().numpy(), dc.gemm_ref(_np(d), x.float().cpu().numpy(), saturated=False))
    assert mx <= 1e-2 and med <= 2e-3, (mx, med)
