"""GPU parity of the chunked few-row fused decode+GEMM (bf16x_gemm_chunks in
the C ABI: 1 <= M <= 64, in_f % 256 == 0; the bf16x_gemm_fused.py:97-114
contract at its small blocks) and of its chunk plan against the oracle.

fp32 activations that are exactly bf16 give y = the fp32 accumulation of one
pass, held to 1e-3 of the float64 product (a dropped or misplaced term, about
1/sqrt(in_f) of an output, fails it).  Rows of I pick W columns bit for bit,
which pins the LDS tile layout, the MFMA operand and result layouts, the
cross-wave sum and every overflow patch, the loop for crowded chunks
included.  The cases reach every kernel shape the launcher picks: one,
two and four 16-row tiles, chunks of 256, 512 and 1024 columns, one or two
token tiles per wave and two token groups."""

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


def _chunks(bx, x, g, out_f, in_f, plan, y_dtype=None):
    """bf16x_gemm_chunks through the C ABI: y[M, out_f] in bf16 or fp32."""
    L = bx._lib.lib()
    yd = bx._lib.BF16 if y_dtype is None else y_dtype
    y = torch.empty(x.shape[0], out_f, dtype=torch.bfloat16 if yd == bx._lib.BF16 else torch.float32, device=DEV)
    st = L.bf16x_gemm_chunks(x.data_ptr(), bx._lib.BF16, x.shape[0], g["sign_packed"].data_ptr(),
                             g["sign_packed"].numel(), g["mant_packed"].data_ptr(), g["mant_packed"].numel(),
                             g["delta_packed"].data_ptr(), g["delta_packed"].numel(), g["emax"].data_ptr(),
                             g["emax"].numel(), bx._lib.ptr(plan.cplan()[0]) if plan is not None else None,
                             bx._lib.ptr(plan.cplan()[1]) if plan is not None else None, out_f, in_f, 16,
                             bx._lib.EXACT if plan is not None else bx._lib.SATURATED, y.data_ptr(), yd,
                             bx._lib.stream_of(x.device))
    bx._lib.check(st, "bf16x_gemm_chunks")
    return y


def _cplan_ref(plan, out_f, in_f):
    """The chunk plan from the row plan on the host: the entries of every
    (256-column chunk p, row r) in that order, re-encoded as (r & 255) << 24
    | (column - 256 p) << 16 | bits, and the offset of each (p, r) run."""
    off = plan.tile_off.cpu().numpy().astype(np.int64)
    ent = plan.tile_ent.cpu().numpy().view(np.uint32).astype(np.int64)[:plan.n_fix]
    C5 = in_f // 256
    runs = [[] for _ in range(C5 * out_f)]
    for r in range(out_f):
        for v in ent[off[r]:off[r + 1]]:
            col = v >> 16
            p = col // 256
            runs[p * out_f + r].append(((r & 255) << 24) | ((col - 256 * p) << 16) | (v & 0xFFFF))
    cp_off = np.zeros(C5 * out_f + 1, np.int64)
    cp_off[1:] = np.cumsum([len(u) for u in runs])
    cp_ent = np.array([v for u in runs for v in u], np.int64)
    return cp_off, cp_ent


@pytest.mark.parametrize("out_f,in_f", [(300, 2048), (77, 768), (1, 256)])
def test_cplan_matches_host(bx, out_f, in_f):
    _, _, _, plan = _weight(bx, out_f, in_f, seed=out_f)
    cp_off, cp_ent = plan.cplan()
    got_off = cp_off.cpu().numpy().view(np.uint32).astype(np.int64)
    got_ent = cp_ent.cpu().numpy().view(np.uint32).astype(np.int64)
    assert got_off.size == bx._lib.lib().bf16x_cplan_size(out_f, in_f) == out_f * (in_f // 256) + 1
    assert got_ent.size == plan.n_fix + 1
    ref_off, ref_ent = _cplan_ref(plan, out_f, in_f)
    assert np.array_equal(got_off, ref_off)
    assert np.array_equal(got_ent[:plan.n_fix], ref_ent)


# (M, out_f, in_f, chunk_atoms override): rows per workgroup and token count
# pick the kernel shape (rt 16-row tiles, ca atoms per chunk, token groups x
# tiles per wave), see bf16x_gemm_chunks
CASES = [
    (3, 1000, 2048, None),     # rt 1, ca 32, 1 x 1
    (20, 700, 4096, None),     # rt 1, ca 32, 1 x 2
    (40, 900, 2048, None),     # rt 2 (16 rows used), ca 16, 2 x 2
    (17, 5000, 1536, None),    # rt 2, ca 16, 1 x 2
    (64, 6000, 1024, None),    # rt 2, ca 16, 2 x 2
    (9, 9000, 512, None),      # rt 4, ca 16, 1 x 1
    (33, 9000, 768, None),     # rt 4, ca 8, 2 x 2
    (64, 16400, 256, None),    # rt 4, ca 8, 2 x 2, one chunk, 257 workgroups
    (30, 12000, 2048, 8),      # rt 4, ca 8 (override), 1 x 2
    (5, 300, 14336, None),     # rt 1, ca 32, 14 chunks
]


@pytest.mark.parametrize("M,out_f,in_f,ca", CASES)
def test_chunks_fp32_product(bx, M, out_f, in_f, ca):
    print("chunks fp32", M, out_f, in_f, ca, flush=True)
    bits, d, g, plan = _weight(bx, out_f, in_f, seed=M + out_f)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
    dn = _np(d)
    with bx.tuning(**({"chunk_atoms": ca} if ca else {})):
        for p, sat in ((plan, False), (None, True)):
            y = _chunks(bx, x.to(DEV), g, out_f, in_f, p, bx._lib.F32)
            assert y.shape == (M, out_f)
            mx, med = dc.rel_err(y.cpu().numpy(), dc.gemm_ref(dn, x.double().numpy(), saturated=sat))
            assert mx <= 1e-3 and med <= 1e-6, (sat, mx, med)
            yb = _chunks(bx, x.to(DEV), g, out_f, in_f, p)
            check_tol(yb.float().cpu().numpy(), dc.gemm_ref(dn, x.float().numpy(), saturated=sat))


@pytest.mark.parametrize("M,out_f,in_f", [(32, 136, 2048), (64, 9000, 512), (48, 520, 1024), (16, 8300, 1024)])
def test_chunks_identity_is_bit_exact(bx, M, out_f, in_f):
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
            y = _chunks(bx, eye.to(DEV), g, out_f, in_f, p)
            got = y.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)[:cols].T.copy()
            got[(got & 0x7F80) == 0] = 0
            assert np.array_equal(got, ref[:, start:start + cols]), (start, p is None)


@pytest.mark.parametrize("out_f,M", [(40, 16), (9000, 64)])
def test_chunks_dense_overflow(bx, out_f, M):
    """Rows with about 90 plan entries per 256-column chunk, past the slots a
    wave preloads per row: the loop that patches the rest."""
    in_f = 1024
    rng = np.random.default_rng(9)
    bits = dc.bench_weight_bits(out_f, in_f, seed=9)
    tiny = rng.random(bits.shape) < 0.35
    bits[tiny] = (bits[tiny] & 0x807F) | 0x0080
    d = bx.bf16x_quantize(bits_tensor(bits))
    plan = bx.build_plan_host(d, device=DEV)
    assert plan.n_fix > out_f * 300
    g = to_dev(d)
    ref_bits = bits.copy()
    ref_bits[(ref_bits & 0x7F80) == 0] = 0
    for start in range(0, in_f, M):
        eye = torch.zeros(M, in_f, dtype=torch.bfloat16)
        eye[torch.arange(M), start + torch.arange(M)] = 1
        y = _chunks(bx, eye.to(DEV), g, out_f, in_f, plan)
        got = y.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).T.copy()
        got[(got & 0x7F80) == 0] = 0
        assert np.array_equal(got, ref_bits[:, start:start + M]), start
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    y = _chunks(bx, x.to(DEV), g, out_f, in_f, plan, bx._lib.F32)
    mx, med = dc.rel_err(y.cpu().numpy(), dc.gemm_ref(_np(d), x.double().numpy(), saturated=False))
    assert mx <= 1e-3 and med <= 1e-6, (mx, med)


def test_chunks_rejects_other_shapes(bx):
    """M outside 1..64 and in_f not a multiple of 256 return BF16X_ESHAPE
    (streams long enough for the shape, so only the shape is wrong)."""
    out_f = 64
    L = bx._lib.lib()
    for M, in_f in ((65, 2048), (0, 2048), (4, 128), (4, 1056)):
        _, _, g, _ = _weight(bx, out_f, in_f, seed=2, specials=False)
        x = torch.zeros(max(M, 1), in_f, dtype=torch.bfloat16, device=DEV)
        y = torch.empty(max(M, 1), out_f, dtype=torch.bfloat16, device=DEV)
        st = L.bf16x_gemm_chunks(x.data_ptr(), bx._lib.BF16, M, g["sign_packed"].data_ptr(),
                                 g["sign_packed"].numel(), g["mant_packed"].data_ptr(), g["mant_packed"].numel(),
                                 g["delta_packed"].data_ptr(), g["delta_packed"].numel(), g["emax"].data_ptr(),
                                 g["emax"].numel(), None, None, out_f, in_f, 16, bx._lib.SATURATED, y.data_ptr(),
                                 bx._lib.BF16, bx._lib.stream_of(x.device))
        assert st == bx._lib.ESHAPE, (M, in_f, st)


@pytest.mark.parametrize("M,out_f,in_f", [(24, 600, 2048), (64, 9000, 1024)])
def test_chunks_through_bf16x_gemm(bx, M, out_f, in_f):
    """bf16x_gemm (fused and auto) dispatches these shapes to the chunked
    kernel; fp32 activations are split into two bf16 passes (x = hi + lo),
    so the product is held against the float64 product of hi + lo (16
    significant bits of x): what remains is the fp32 accumulation."""
    assert bx.ops._use_chunks(M, out_f, in_f, torch.device(DEV))
    bits, d, g, plan = _weight(bx, out_f, in_f, seed=M + 3)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(M + 3))
    hi = x.to(torch.bfloat16)
    x_split = hi.double() + (x - hi.float()).to(torch.bfloat16).double()
    y_ref = dc.gemm_ref(_np(d), x_split.numpy(), saturated=False)
    for path in ("fused", "auto"):
        y = bx.bf16x_gemm(x.to(DEV), g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"], out_f, in_f,
                          plan=plan, path=path)
        assert y.dtype == torch.float32
        mx, med = dc.rel_err(y.cpu().numpy(), y_ref)
        assert mx <= 1e-3 and med <= 1e-5, (path, mx, med)


@pytest.mark.parametrize("out_f,in_f", [(14336, 4096), (4096, 4096), (4096, 14336)])
@pytest.mark.parametrize("M", [17, 64])
def test_chunks_full_size(bx, M, out_f, in_f):
    """Configuration-3 projection shapes, exact, against the fp32 product of
    the original weight on the device."""
    print("chunks full", M, out_f, in_f, flush=True)
    bits = dc.bench_weight_bits(out_f, in_f, seed=1)
    w = bits_tensor(bits)
    d = bx.bf16x_quantize(w)
    g = to_dev(d)
    plan = bx.build_plan_host(d, device=DEV)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(DEV)
    y_ref = (x.float() @ w.to(DEV).float().t()).double().cpu().numpy()
    y = _chunks(bx, x, g, out_f, in_f, plan)
    mx, med = check_tol(y.float().cpu().numpy(), y_ref)
    print("chunks full-size rel err max %.2e median %.2e" % (mx, med), flush=True)
