"""The reference's own BF16X self-test (opqk_linear.py:470-511, "Mode2:
BF16X" and its forward line) at its configuration, on the GPU path.

The weight is built exactly as there: torch.manual_seed(0), nn.Linear(5376,
28672) (CPU init), weight x 0.13, 0.5 % of the entries (torch.randperm) x
randn x 8.  The reference prints the share of bf16-exact weights after a
round trip ("should = 100") and the forward's norm-relative error against
F.linear in bf16 for a random x of 4 rows; here both become assertions: the
decode is bit-exact (100 %), and the module's forward (the fused GEMM at 4
rows, then the bias added in bf16 as the reference's forward adds it) is
within the north-star tolerance of an fp64 product plus that addition's
rounding, and at bf16 noise against F.linear."""

import pytest
import torch

from tests.test_gpu_modules import check_biased

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module")
def bx():
    import bfloat16x_amd as m
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return m


@pytest.fixture(scope="module")
def selftest_linear():
    torch.manual_seed(0)
    lin = torch.nn.Linear(5376, 28672, bias=True)
    with torch.no_grad():
        lin.weight.mul_(0.13)
        idx = torch.randperm(lin.weight.numel())[: lin.weight.numel() // 200]
        lin.weight.reshape(-1)[idx] *= torch.randn(len(idx)) * 8
    return lin


def test_reference_selftest_round_trip_and_forward(bx, selftest_linear):
    print("reference self-test 28672x5376", flush=True)
    lin = selftest_linear
    w16 = lin.weight.data.to(torch.bfloat16)
    # device encoder (the same bytes as the host encoder, test_gpu_encode.py)
    d = bx.bf16x_quantize(lin.weight.data.to(DEV))
    n = lin.weight.numel()
    n_ovf = int(d["delta_ovf_idx"].numel())
    bpw = (7 * n + 3 * n + n + 40 * n_ovf + 8 * ((n + 15) // 16)) / n     # opqk_linear.py:461-467
    q = bx.BF16XLinear.from_packed(d, tile=1024, bias=lin.bias.data, device=DEV)
    dec = q.decoded_weight().to(torch.bfloat16)
    exact = (dec.cpu().view(torch.int16) == w16.view(torch.int16)).float().mean().item() * 100
    print(f"BPW {bpw:.2f} | bf16 exact {exact:.2f} % (should be 100)", flush=True)
    assert exact == 100.0
    # forward, as the reference's: bf16 x of 4 rows against F.linear in bf16
    x = torch.randn(4, 5376, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(DEV)
    wb, bb = w16.to(DEV), lin.bias.data.to(torch.bfloat16).to(DEV)
    y_orig = torch.nn.functional.linear(x, wb, bb).float()
    with torch.no_grad():
        y = q(x).float()
    rel = ((y_orig - y).norm() / y_orig.norm()).item()
    print(f"BF16X forward relative error {rel:.2e}", flush=True)
    assert rel <= 4e-3                                       # two bf16 roundings of the same product
    # elementwise: the product's tolerance plus the bf16 rounding of the bias
    # addition, which the reference's forward also does in bf16
    # (opqk_linear.py:401-403)
    xw = (x.double() @ wb.double().t().contiguous()).cpu().numpy()
    check_biased(y, xw, bb)
