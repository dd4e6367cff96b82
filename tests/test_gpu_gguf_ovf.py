"""GPU tests of the GGUF lossless side table: the decode with the table
returns the original bf16 bits of every element (including rows with more
than 64 entries in one 2048-column pass and weights wider than one pass);
the GEMV and GEMM over the lossless weight match the exact product; a table
that fails the host check is refused."""
import numpy as np
import pytest
import torch

from oracle import gguf_codec as go
from tests.test_gguf_ovf_host import selftest_weights
from tests.test_gpu_dict import DEV, check_tol

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def g():
    from bfloat16x_amd import gguf
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return gguf


def dense_overflow(rows, cols, seed):
    """Student-t weights with most of a few rows' elements far below their
    half-block max: many entries per row and per pass."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_t(3, size=(rows, cols)) * 0.015).astype(np.float32)
    w[1, :] *= 1e-4
    w[1, ::16] = 1.0                       # one large element per half: the rest clamp
    w[2, 100:3000] = 1e-30
    return w


# ("dense", (4100, 4224)): the long-row GEMV (3 passes of 64 blocks), two rows
# per wave, rows 1 and 2 with more entries than the read-ahead batches
CASES = [("selftest", (256, 512)), ("selftest", (300, 576)), ("dense", (8, 4096)), ("dense", (5, 8192)),
         ("selftest", (64, 2080)), ("dense", (4100, 4224))]


def weights(kind, shape, seed):
    return selftest_weights(shape, seed) if kind == "selftest" else dense_overflow(*shape, seed)


@torch.no_grad()
@pytest.mark.parametrize("kind,shape", CASES)
def test_lossless_decode_bit_exact(g, kind, shape):
    w = weights(kind, shape, 4)
    bits = go.fp32_to_bf16_bits(w)
    packed = g.quantize_blocks(w)
    blob = g.pack_ovf(w)
    rows, ro, _, _ = g.unpack_ovf(blob)
    t = g.device_ovf(blob, packed, DEV)
    blocks = g.device_blocks(packed, DEV)
    for dtype in (torch.bfloat16, torch.float32):
        out = g.gguf_decode(blocks, *shape, dtype=dtype, ovf=t)
        got = go.fp32_to_bf16_bits(out.float().cpu().numpy())
        assert np.array_equal(got, bits), (dtype, int((got != bits).sum()))
    assert np.array_equal(go.fp32_to_bf16_bits(g.dequantize_lossless(packed, blob)), bits.reshape(-1))
    if kind == "dense":
        assert int(np.diff(ro).max()) > 64
    # without the table: the plain decode, different exactly on the table's elements
    plain = go.fp32_to_bf16_bits(g.gguf_decode(blocks, *shape, dtype=torch.float32).cpu().numpy())
    assert np.array_equal(plain != bits, g.ovf_overflow_mask(w))


@torch.no_grad()
@pytest.mark.parametrize("kind,shape", CASES)
def test_lossless_gemv_gemm(g, kind, shape):
    w = weights(kind, shape, 5)
    wb = go.bf16_bits_to_fp32(go.fp32_to_bf16_bits(w)).astype(np.float64).reshape(shape)
    packed = g.quantize_blocks(w)
    t = g.device_ovf(g.pack_ovf(w), packed, DEV)
    blocks = g.device_blocks(packed, DEV)
    x = torch.randn(shape[1], generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    ref = wb @ x.double().numpy()
    for od in (torch.float32, torch.bfloat16):
        y = g.gguf_gemv(x.to(DEV), blocks, *shape, out_dtype=od, ovf=t)
        check_tol(y.float().cpu().numpy(), ref)
    xm = torch.randn(7, shape[1], generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    check_tol(g.gguf_gemm(xm.to(DEV), blocks, *shape, ovf=t).float().cpu().numpy(), xm.double().numpy() @ wb.T)
    if shape[1] % 64 == 0:
        # the fused GEMM with the table's step-major plan (two row counts:
        # one partial tile, and more than one 256-row tile)
        for M in (7, 300):
            xm = torch.randn(M, shape[1], generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
            y = g.gguf_gemm_fused(xm.to(DEV), blocks, *shape, out_dtype=torch.float32, ovf=t)
            check_tol(y.cpu().numpy(), xm.double().numpy() @ wb.T)


# Whole-K tiles in full rounds and the last round's tiles split over K (the
# resident block count forced to 4): 520 x 300 rows x columns is 3 x 3 = 9
# tiles, run as 8 whole tiles and one tile in 4 K ranges, with the table's
# plan (lossless) and without it.
@pytest.mark.parametrize("kind,shape", [("dense", (300, 4096)), ("selftest", (300, 1024))])
def test_gemm_fused_mixed_rounds(g, tune, kind, shape):
    print("gguf gemm mixed rounds", kind, shape, flush=True)
    tune(gemm_ws_resident=4)
    w = weights(kind, shape, 9)
    wb = go.bf16_bits_to_fp32(go.fp32_to_bf16_bits(w)).astype(np.float64).reshape(shape)
    packed = g.quantize_blocks(w)
    wnl = go.dequantize_blocks(packed).astype(np.float64).reshape(shape)
    t = g.device_ovf(g.pack_ovf(w), packed, DEV)
    blocks = g.device_blocks(packed, DEV)
    xm = torch.randn(520, shape[1], generator=torch.Generator().manual_seed(11)).to(torch.bfloat16)
    for ovf, ref in ((t, wb), (None, wnl)):
        y = g.gguf_gemm_fused(xm.to(DEV), blocks, *shape, out_dtype=torch.float32, ovf=ovf)
        check_tol(y.cpu().numpy(), xm.double().numpy() @ ref.T)


def test_tampered_table_refused(g):
    from bfloat16x_amd import _lib
    w = selftest_weights((16, 256), 8)
    packed = g.quantize_blocks(w)
    blob = bytearray(g.pack_ovf(w))
    off = 8 + 4 * 17                    # first entry: flip the sign bit of its bf16 bits
    blob[off + 3] ^= 0x80
    with pytest.raises(_lib.Bf16xError):
        g.device_ovf(bytes(blob), packed, DEV)
