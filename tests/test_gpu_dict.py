"""GPU parity of the packed-dict kernels against the oracle (bit-exact decode,
GEMV within the tolerance of the north star), through the C ABI."""
import numpy as np
import pytest
import torch

from oracle import dict_codec as dc

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
SPECIALS = np.array([0x0000, 0x8000, 0x0001, 0x807F, 0x7F80, 0xFF80, 0x7FC1, 0x3F80, 0x7F7F, 0x0080,
                     0x3C00, 0x4300], np.uint16)


@pytest.fixture(scope="module")
def bx():
    import bfloat16x_amd as m
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return m


def to_dev(d):
    return {k: (torch.as_tensor(v).to(DEV) if isinstance(v, (np.ndarray, torch.Tensor)) else v)
            for k, v in d.items()}


def bits_tensor(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def with_specials(bits, seed, k=40):
    b = bits.copy().reshape(-1)
    rng = np.random.default_rng(seed)
    b[rng.choice(b.size, min(k, b.size), replace=False)] = rng.choice(SPECIALS, min(k, b.size))
    return b.reshape(bits.shape)


def gpu_bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("shape", [(2048, 1536), (64, 4096), (16, 14336), (2, 70016), (7, 9), (5, 13), (33, 40),
                                   (3, 96)])
def test_decode_exact_and_saturated(bx, shape):
    print("decode", shape, flush=True)
    bits = with_specials(dc.bench_weight_bits(*shape, seed=0), seed=1)
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    plan = bx.build_plan_host(d, check=2, device=DEV)
    ex = bx.bf16x_decode(g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], *shape, plan=plan)
    torch.cuda.synchronize()
    assert np.array_equal(gpu_bits(ex), bits)
    sat = bx.bf16x_decode(g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], *shape)
    assert np.array_equal(gpu_bits(sat), dc.decode_saturated({k: (v.numpy() if isinstance(v, torch.Tensor) else v)
                                                              for k, v in d.items()}))


def test_decode_reference_call_pattern(bx):
    """bf16x_decode_triton(sign.cuda(), ..., ovf_idx_cpu, ovf_val_cpu): table on
    the host, streams on the GPU; the plan is built once and cached."""
    shape = (256, 1536)
    bits = dc.bench_weight_bits(*shape, seed=9)
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    args = (g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], *shape,
            d["delta_ovf_idx"], d["delta_ovf_val"])
    from bfloat16x_amd import ops
    n0 = len(ops._PLANS.d)
    w1 = bx.bf16x_decode_triton(*args)
    w2 = bx.bf16x_decode_triton(*args)
    assert len(ops._PLANS.d) == n0 + 1
    assert np.array_equal(gpu_bits(w1), bits) and np.array_equal(gpu_bits(w2), bits)
    # padded streams (the reference's _pad1) are accepted
    pad = lambda t: torch.cat([t, torch.zeros(1, dtype=t.dtype, device=t.device)])
    w3 = bx.bf16x_decode(pad(g["sign_packed"]), pad(g["mant_packed"]), pad(g["delta_packed"]), g["emax"],
                         *shape, d["delta_ovf_idx"], d["delta_ovf_val"])
    assert np.array_equal(gpu_bits(w3), bits)


def check_tol(y, y_ref, max_tol=1e-2, med_tol=2e-3):
    mx, med = dc.rel_err(y, y_ref)
    assert mx <= max_tol and med <= med_tol, (mx, med)
    return mx, med


# (2103, 14336): rows split over 4 waves with 4 row groups per workgroup and a
# ragged last workgroup; fp32 x above 16384 columns (16, 28672) runs the
# generic kernel (x read from memory, not staged in LDS)
@pytest.mark.parametrize("shape", [(48, 1536), (2048, 1536), (256, 4096), (40, 14336), (16, 28672), (2103, 14336)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
def test_gemv_exact(bx, shape, xdt):
    print("gemv", shape, xdt, flush=True)
    bits = dc.bench_weight_bits(*shape, seed=2)
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    plan = bx.build_plan_host(d, device=DEV)
    x = torch.randn(shape[1], generator=torch.Generator().manual_seed(1)).to(xdt)
    y = bx.bf16x_gemv(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], *shape,
                      plan=plan)
    assert y.dtype == torch.bfloat16 and y.shape == (shape[0],)
    y_ref = dc.bits_to_f32(bits).astype(np.float64) @ x.float().numpy().astype(np.float64)
    check_tol(y.float().cpu().numpy(), y_ref)


def test_gemv_saturated_and_fp16(bx):
    shape = (128, 4096)
    bits = dc.bench_weight_bits(*shape, seed=3)
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    dn = {k: (v.numpy() if isinstance(v, torch.Tensor) else v) for k, v in d.items()}
    x = torch.randn(shape[1], generator=torch.Generator().manual_seed(2))
    for xdt in (torch.bfloat16, torch.float16):
        xx = x.to(xdt)
        y = bx.bf16x_gemv(xx.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], *shape)
        y_ref = dc.gemm_ref(dn, xx.float().numpy()[None], saturated=True)[0]
        check_tol(y.float().cpu().numpy(), y_ref)


def test_fused_gemv_reference_csr(bx):
    """bf16x_fused_gemv with the reference's per-row CSR (bf16x_fused.py:165-179)."""
    shape = (512, 4096)
    bits = dc.bench_weight_bits(*shape, seed=4)
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    idx = d["delta_ovf_idx"].to(torch.int64)
    val = d["delta_ovf_val"].to(torch.int64)
    keep = val > 7
    idx, val = idx[keep], val[keep]
    rows, k = idx // shape[1], idx % shape[1]
    counts = torch.bincount(rows, minlength=shape[0])
    oloff = torch.zeros(shape[0] + 1, dtype=torch.int32)
    oloff[1:] = counts.cumsum(0).to(torch.int32)
    x = torch.randn(shape[1], generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    y = bx.bf16x_fused_gemv(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"],
                            k.to(torch.int32).to(DEV), val.to(torch.int32).to(DEV), oloff.to(DEV), *shape)
    y_ref = dc.bits_to_f32(bits).astype(np.float64) @ x.float().numpy().astype(np.float64)
    check_tol(y.float().cpu().numpy(), y_ref)


def test_ops_reject_mismatched_buffers(bx):
    """The wrappers hand raw pointers to the kernels, so every caller-supplied
    buffer is checked first: an output too small or on the CPU, a plan built
    for another shape, a reference CSR of the wrong dtype or length.  Each is
    refused on the host before any launch."""
    shape = (256, 1024)
    bits = dc.bench_weight_bits(*shape, seed=21)
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    streams = (g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"])
    plan = bx.build_plan_host(d, device=DEV)
    x = torch.randn(shape[1], generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(DEV)
    with pytest.raises(ValueError):
        bx.bf16x_gemv(x, *streams, *shape, plan=plan, out=torch.empty(shape[0] - 1, dtype=torch.bfloat16,
                                                                       device=DEV))
    with pytest.raises(ValueError):
        bx.bf16x_gemv(x, *streams, *shape, plan=plan, out=torch.empty(shape[0], dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        bx.bf16x_decode(*streams, *shape, plan=plan, out=torch.empty(shape[0] * shape[1], dtype=torch.bfloat16))
    other = bx.build_plan_host(bx.bf16x_quantize(bits_tensor(dc.bench_weight_bits(128, 1024, seed=3))), device=DEV)
    for call in (lambda: bx.bf16x_gemv(x, *streams, *shape, plan=other),
                 lambda: bx.bf16x_decode(*streams, *shape, plan=other),
                 lambda: bx.bf16x_gemm(x.reshape(1, -1).repeat(80, 1), *streams, *shape, plan=other)):
        with pytest.raises(ValueError):
            call()
    k = torch.zeros(4, dtype=torch.int64, device=DEV)
    v = torch.full((4,), 9, dtype=torch.int32, device=DEV)
    off = torch.zeros(shape[0] + 1, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):
        bx.bf16x_fused_gemv(x, *streams, k, v, off, *shape)               # int64 columns
    with pytest.raises(ValueError):
        bx.bf16x_fused_gemv(x, *streams, k.to(torch.int32), v, off[:-1], *shape)   # short offsets
    # the calls that pass still agree with the oracle
    y = bx.bf16x_gemv(x, *streams, *shape, plan=plan, out=torch.empty(shape[0], dtype=torch.bfloat16, device=DEV))
    check_tol(y.float().cpu().numpy(), dc.bits_to_f32(bits).astype(np.float64) @ x.float().cpu().numpy())


def test_fused_gemv_csr_offsets_are_clamped(bx):
    """A reference CSR whose offsets point past its entries (a malformed
    table) cannot make a kernel read outside the entry arrays: the plan keeps
    the offsets in [0, n], and the rows whose runs were cut lose only their
    corrections."""
    shape = (64, 1024)
    bits = dc.bench_weight_bits(*shape, seed=22)
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    x = torch.randn(shape[1], generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(DEV)
    k = torch.tensor([3, 7], dtype=torch.int32, device=DEV)
    v = torch.tensor([9, 10], dtype=torch.int32, device=DEV)
    off = torch.full((shape[0] + 1,), 2, dtype=torch.int32, device=DEV)
    off[0] = 0
    off[-1] = 1 << 20                                                    # past the two entries
    plan = bx.ops.plan_for_csr(k, v, off, g["sign_packed"], g["mant_packed"], g["emax"], *shape)
    assert int(plan.tile_off.max()) == 2
    y = bx.bf16x_gemv(x, g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], *shape, plan=plan)
    assert torch.isfinite(y.float()).all()


@pytest.mark.parametrize("out_f,in_f", [(4100, 6144), (40, 4128), (1030, 16384)])
def test_gemv_long_rows_dense_overflow(bx, out_f, in_f):
    """Rows longer than 4096 columns (the one-wave-per-row kernel) with far
    more plan entries than the batches read ahead per row: 30 % of the
    elements are tiny (delta >= 7 next to normal values), so every row parks
    its sum and finishes its entries after the wave's last row; ragged row
    counts, a partial last pass (4128 columns), one and two rows per wave."""
    bits = dc.bench_weight_bits(out_f, in_f, seed=in_f)
    rng = np.random.default_rng(in_f)
    tiny = rng.random(bits.shape) < 0.3
    bits[tiny] = (bits[tiny] & 0x807F) | 0x0080
    d = bx.bf16x_quantize(bits_tensor(bits))
    plan = bx.build_plan_host(d, device=DEV)
    assert plan.n_fix > out_f * (in_f // 2048) * 64
    g = to_dev(d)
    x = torch.randn(in_f, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    y = bx.bf16x_gemv(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                      plan=plan)
    y_ref = dc.bits_to_f32(bits).astype(np.float64) @ x.float().numpy().astype(np.float64)
    check_tol(y.float().cpu().numpy(), y_ref)
    ys = bx.bf16x_gemv(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f)
    ys_ref = dc.bits_to_f32(dc.decode_saturated({k: (v.numpy() if isinstance(v, torch.Tensor) else v)
                                                 for k, v in d.items()})).astype(np.float64) @ \
        x.float().numpy().astype(np.float64)
    check_tol(ys.float().cpu().numpy(), ys_ref)


def test_full_size_roundtrip_and_gemv(bx):
    """14336x4096 at full size: encode -> exact decode is the identity on the
    original bits, and the GEMV matches fp32 matmul of the decoded weight."""
    shape = (14336, 4096)
    print("full size", shape, flush=True)
    bits = dc.bench_weight_bits(*shape, seed=0)
    w = bits_tensor(bits)
    d = bx.bf16x_quantize(w)
    g = to_dev(d)
    plan = bx.build_plan_host(d, device=DEV)
    wd = w.to(DEV)
    dec = bx.bf16x_decode(g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], *shape, plan=plan)
    assert torch.equal(dec.view(torch.int16), wd.view(torch.int16))
    x = torch.randn(shape[1], generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(DEV)
    y = bx.bf16x_gemv(x, g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], *shape, plan=plan)
    y_ref = (wd.float() @ x.float()).double().cpu().numpy()
    mx, med = check_tol(y.float().cpu().numpy(), y_ref)
    print("full-size gemv rel err max %.2e median %.2e" % (mx, med), flush=True)
