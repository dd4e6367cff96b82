"""The allocation-free GGUF GEMV (bf16x_gguf_gemv_noalloc, a fixed device
scratch array inside the library) against bf16x_gguf_gemv with a caller
workspace, through the C ABI: two calls in a row, the second on a smaller
input, on both the x-staging kernel (short rows, which uses the scratch) and
the long-row kernel; and the refusal of in_f beyond the scratch."""
import numpy as np
import pytest
import torch

from oracle import gguf_codec as gc

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _call(L, noalloc, x, blocks, out_f, in_f, ws=None):
    from bfloat16x_amd import _lib
    y = torch.empty(out_f, dtype=torch.bfloat16, device=DEV)
    if noalloc:
        st = L.bf16x_gguf_gemv_noalloc(x.data_ptr(), _lib.BF16, blocks.data_ptr(), blocks.numel(), out_f, in_f,
                                       y.data_ptr(), _lib.BF16, _lib.stream_of(x.device))
    else:
        st = L.bf16x_gguf_gemv(x.data_ptr(), _lib.BF16, blocks.data_ptr(), blocks.numel(), out_f, in_f, y.data_ptr(),
                               _lib.BF16, ws.data_ptr(), ws.numel() * 4, _lib.stream_of(x.device))
    return st, y


@pytest.mark.parametrize("shapes", [((1024, 4096), (200, 1024)), ((256, 8192), (96, 6144))])
def test_gguf_gemv_noalloc_matches_workspace_entry(shapes):
    import bfloat16x_amd as bx
    from bfloat16x_amd import _lib
    L = _lib.lib()
    for out_f, in_f in shapes:                     # the second call is smaller
        print("noalloc gguf gemv", out_f, in_f, flush=True)
        w = gc.student_t_weights(out_f, in_f, seed=out_f + in_f)
        blocks = bx.gguf.device_blocks(bx.gguf.quantize_blocks(w), DEV)
        x = torch.randn(in_f, generator=torch.Generator().manual_seed(in_f)).to(torch.bfloat16).to(DEV)
        ws = torch.empty((int(L.bf16x_gguf_gemv_workspace(in_f)) + 15) // 16 * 4, dtype=torch.int32, device=DEV)
        st0, y0 = _call(L, False, x, blocks, out_f, in_f, ws)
        st1, y1 = _call(L, True, x, blocks, out_f, in_f)
        torch.cuda.synchronize()
        assert st0 == 0 and st1 == 0, (st0, st1)
        # the same kernels on the same inputs: bit-identical outputs
        assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
        # and within the north-star tolerance of the oracle's product
        ref = gc.dequantize_blocks(bx.gguf.quantize_blocks(w)).astype(np.float64) @ x.float().cpu().numpy()
        err = np.abs(y1.float().cpu().numpy() - ref) / np.maximum(np.abs(ref), 1e-3 * np.sqrt(np.mean(ref ** 2)))
        assert err.max() <= 1e-2 and np.median(err) <= 2e-3


def test_gguf_gemv_noalloc_refuses_oversize():
    from bfloat16x_amd import _lib
    L = _lib.lib()
    in_f = 65536 + 32
    x = torch.zeros(in_f, dtype=torch.bfloat16, device=DEV)
    blocks = torch.zeros(in_f // 32 * 46, dtype=torch.uint8, device=DEV)
    st, _ = _call(L, True, x, blocks, 1, in_f)
    assert st == _lib.ECAPACITY
