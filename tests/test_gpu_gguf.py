"""GPU parity of the GGUF half-block kernels against the oracle
(oracle/gguf_codec.py, pinned by the reference's golden vectors): bit-exact
decode, GEMV / GEMM within the north-star tolerance, and configuration 5's
70B-layer shapes end to end."""
import numpy as np
import pytest
import torch

from oracle import dict_codec as dc
from oracle import gguf_codec as gc
from tests.test_gpu_dict import DEV, check_tol

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def bx():
    import bfloat16x_amd as m
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return m


def _dev_decode_bits(bx, blocks_np, out_f, in_f):
    b = bx.gguf.device_blocks(blocks_np, DEV)
    y = bx.gguf.gguf_decode(b, out_f, in_f)
    return y.view(torch.int16).cpu().numpy().view(np.uint16)


def test_decode_golden_and_junk(bx, golden):
    blk = golden["gguf_blocks"]                       # (4, 2, 46): rows of 64
    assert np.array_equal(_dev_decode_bits(bx, blk, 4, 64), gc.fp32_to_bf16_bits(golden["gguf_dequant"]))
    junk = golden["gguf_junk_blocks"]                 # arbitrary bytes, 3 blocks (odd: padded)
    got = _dev_decode_bits(bx, junk, 1, 96).reshape(-1)
    assert np.array_equal(got, golden["gguf_junk_dequant"].view(np.uint32).reshape(-1) >> 16)
    st = golden["gguf_selftest_blocks"]               # (32, 16, 46)
    assert np.array_equal(_dev_decode_bits(bx, st, 32, 512).reshape(32, 512),
                          golden["gguf_selftest_dequant"].view(np.uint32) >> 16)


@pytest.mark.parametrize("shape", [(1, 32), (3, 96), (5, 4096), (64, 2080), (33, 8192)])
def test_decode_random_blocks_bit_exact(bx, shape):
    """Random bytes exercise every code, emax below the floor and the zero
    marker; odd block counts exercise the tail padding."""
    nb = shape[0] * shape[1] // 32
    rng = np.random.default_rng(nb)
    blocks = rng.integers(0, 256, (nb, 46), dtype=np.uint64).astype(np.uint8)
    got = _dev_decode_bits(bx, blocks, *shape).reshape(-1)
    assert np.array_equal(got, gc.dequantize_blocks_bits(blocks).reshape(-1))


def test_dequantize_blocks_api(bx):
    w = gc.student_t_weights(48, 256, seed=1)
    packed = bx.gguf.quantize_blocks(w)
    back = bx.gguf.dequantize_blocks(packed)           # numpy in -> numpy out (GPU decode)
    assert isinstance(back, np.ndarray) and back.shape == w.shape
    assert np.array_equal(back.view(np.uint32), gc.dequantize_blocks(packed).view(np.uint32))
    dev = bx.gguf.dequantize_blocks(torch.from_numpy(packed).to(DEV))
    assert dev.is_cuda and np.array_equal(dev.cpu().numpy().view(np.uint32), back.view(np.uint32))


# (4100, 4224): the long-row GEMV with a partial last pass (132 blocks per
# row), two rows per wave and a ragged last workgroup
@pytest.mark.parametrize("shape", [(256, 4096), (96, 28672), (1000, 1024), (4100, 4224)])
def test_gemv_and_gemm(bx, shape):
    out_f, in_f = shape
    w = gc.student_t_weights(out_f, in_f, seed=2)
    blocks = bx.gguf.quantize_blocks(w)
    wdec = gc.dequantize_blocks(blocks).astype(np.float64).reshape(out_f, in_f)
    b = bx.gguf.device_blocks(blocks, DEV)
    x = torch.randn(in_f, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    for dt in (torch.bfloat16, torch.float32):
        y = bx.gguf.gguf_gemv(x.to(DEV), b, out_f, in_f, out_dtype=dt)
        check_tol(y.float().cpu().numpy(), wdec @ x.double().numpy())
    xm = torch.randn(8, in_f, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    ym = bx.gguf.gguf_gemm(xm.to(DEV), b, out_f, in_f)
    check_tol(ym.float().cpu().numpy(), xm.double().numpy() @ wdec.T)


# fused decode + GEMM: ragged M (rows past M in a 256-row tile), ragged out_f
# (rows past out_f in a 128-row tile), split K (few tiles) and whole K
@pytest.mark.parametrize("shape", [(256, 4096), (1000, 1024), (200, 4224), (96, 28672), (1100, 1024)])
def test_gemm_fused(bx, shape):
    out_f, in_f = shape
    print("gguf gemm fused", shape, flush=True)
    w = gc.student_t_weights(out_f, in_f, seed=5)
    blocks = bx.gguf.quantize_blocks(w)
    wdec = gc.dequantize_blocks(blocks).astype(np.float64).reshape(out_f, in_f)
    b = bx.gguf.device_blocks(blocks, DEV)
    for M in (1, 37, 256, 300):
        xm = torch.randn(M, in_f, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
        ref = xm.double().numpy() @ wdec.T
        for dt in (torch.bfloat16, torch.float32):
            y = bx.gguf.gguf_gemm_fused(xm.to(DEV), b, out_f, in_f, out_dtype=dt)
            assert y.dtype == dt and y.shape == (M, out_f)
            check_tol(y.float().cpu().numpy(), ref)
    # the dispatching entry, leading dims kept: one row (GEMV), the fused
    # GEMM's range, above it (decode + library GEMM)
    for lead in ((1, 1), (3, 1), (2, 150), (1, bx.gguf.GGUF_GEMM_MAX_ROWS_TALL + 1),
                 (1, bx.gguf.GGUF_GEMM_MAX_ROWS + 1)):
        x3 = torch.randn(*lead, in_f, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
        y3 = bx.gguf.gguf_gemm(x3.to(DEV), b, out_f, in_f)
        assert y3.shape == (*lead, out_f) and y3.dtype == torch.bfloat16
        check_tol(y3.float().cpu().numpy().reshape(-1, out_f), x3.double().numpy().reshape(-1, in_f) @ wdec.T)


def test_gemm_fused_refuses(bx):
    from bfloat16x_amd import Bf16xError
    w = gc.student_t_weights(8, 96, seed=1)
    b = bx.gguf.device_blocks(bx.gguf.quantize_blocks(w), DEV)
    x = torch.zeros(4, 96, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(Bf16xError):
        bx.gguf.gguf_gemm_fused(x, b, 8, 96)          # in_f % 64 != 0
    with pytest.raises(ValueError):
        bx.gguf.gguf_gemm_fused(x.float(), b, 8, 96)  # x not bf16


@pytest.mark.parametrize("shape", [(8192, 28672), (28672, 8192)])
def test_config5_full_size(bx, shape):
    """Configuration 5 shapes: encode (C++) -> decode (GPU) keeps sign and
    mantissa of every weight, every clamped weight has exponent 0 and came
    from a code-7 element; the first rows match the oracle bit for bit; the
    GEMV matches fp32 matmul of the decoded weight."""
    out_f, in_f = shape
    print("gguf full size", shape, flush=True)
    w = gc.student_t_weights(out_f, in_f, seed=0)
    bits = bx.gguf.fp32_to_bf16_bits(w)
    blocks = bx.gguf.quantize_blocks(w)
    b = bx.gguf.device_blocks(blocks, DEV)
    dec = bx.gguf.gguf_decode(b, out_f, in_f)
    got = dec.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got[:64], gc.dequantize_blocks_bits(blocks[:64]).reshape(64, in_f))
    mism = got != bits
    assert np.array_equal(got & 0x807F, bits & 0x807F)
    assert np.all((got[mism] & 0x7F80) == 0)
    frac = mism.mean()
    err = np.abs(gc.bf16_bits_to_fp32(got).astype(np.float64) - gc.bf16_bits_to_fp32(bits)).max()
    print(f"clamped fraction {frac:.4%}, max abs reconstruction error {err:.4e}", flush=True)
    assert 0.01 < frac < 0.06
    x = torch.randn(in_f, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(DEV)
    y = bx.gguf.gguf_gemv(x, b, out_f, in_f)
    y_ref = (dec.float() @ x.float()).double().cpu().numpy()
    check_tol(y.float().cpu().numpy(), y_ref)
    # decode + GEMM at M = 512 (the configuration's prefill shape), fused,
    # against an fp64 product of the decoded weight.  Outputs near zero are
    # measured against a floor of 1e-3 rms: there the fp32 accumulation over
    # K = 28672 (1792 sequential MFMA adds, ~2.5e-6 rms each output) is the
    # error, up to ~0.5e-2 of the floor; bf16 outputs add their rounding.
    xm = torch.randn(512, in_f, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(DEV)
    ym_ref = (xm.double() @ dec.double().t()).cpu().numpy()
    y32 = bx.gguf.gguf_gemm_fused(xm, b, out_f, in_f, out_dtype=torch.float32)
    ym = bx.gguf.gguf_gemm(xm, b, out_f, in_f)
    # bf16 output against torch's bf16 matmul on the decoded weight (the
    # north-star comparator) and against the fp64 product; every error is
    # printed before any bound is checked
    yt = torch.nn.functional.linear(xm, dec).float().cpu().numpy()
    e32 = dc.rel_err(y32.cpu().numpy(), ym_ref)
    e16 = dc.rel_err(ym.float().cpu().numpy(), ym_ref)
    e16t = dc.rel_err(ym.float().cpu().numpy(), yt)
    et = dc.rel_err(yt, ym_ref)
    print(f"M=512 rel err (max, median): fp32 out vs fp64 {e32}; bf16 out vs fp64 {e16}; bf16 out vs torch bf16 "
          f"{e16t}; torch bf16 vs fp64 {et}", flush=True)
    for mx, med in (e32, e16, e16t):
        assert mx <= 1e-2 and med <= 2e-3, (e32, e16, e16t)
