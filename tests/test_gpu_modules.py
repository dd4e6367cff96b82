"""GPU tests of the drop-in modules: a deployed model gives the original
model's outputs (exact weight), Bf16xGemmLinear's default gives the
reference's saturated numerics, all Bf16xFused modes agree."""
import copy

import numpy as np
import pytest
import torch
from torch import nn

from oracle import dict_codec as dc
from tests.test_gpu_dict import DEV, check_tol

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def bx():
    import bfloat16x_amd as m
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return m


class MLP(nn.Module):
    def __init__(self, d=512, f=1536):
        super().__init__()
        g = torch.Generator().manual_seed(0)
        self.up = nn.Linear(d, f)
        self.down = nn.Linear(f, d, bias=False)
        for p in self.parameters():
            p.data = (torch.randn(p.shape, generator=g) * 0.03)
        with torch.no_grad():
            self.up.weight.view(-1)[torch.randperm(d * f, generator=g)[: d * f // 100]] *= 30.0

    def forward(self, x):
        return self.down(torch.relu(self.up(x)))


@torch.no_grad()
def _ref_outputs(model, xs):
    """The original model in bf16 on the device (hipBLASLt): the same
    bf16 rounding between layers as the deployed model."""
    m = copy.deepcopy(model).to(torch.bfloat16).to(DEV)
    return [m(x.to(torch.bfloat16)).double().cpu().numpy() for x in xs]


def norm_rel(y, r):
    """||y - r|| / ||r||, the whole-model error measure of the reference
    (opqk_linear.py:510)."""
    y = np.asarray(y, np.float64).reshape(-1)
    r = np.asarray(r, np.float64).reshape(-1)
    return float(np.linalg.norm(y - r) / np.linalg.norm(r))


def check_biased(got, xw, bias):
    """A module output y = bf16(bf16(x.W^T) + bf16(b)) against x.W^T + b:
    the product's elementwise tolerance plus one bf16 rounding of
    |x.W^T| + |b| for the addition done in bf16, as the reference modules
    do it."""
    got = got.float().cpu().numpy()
    b = bias.double().cpu().numpy()
    ref = xw + b
    rms = np.sqrt(np.mean(ref ** 2))
    bound = 1e-2 * np.maximum(np.abs(ref), 1e-3 * rms) + 2.0 ** -8 * (np.abs(xw) + np.abs(b))
    assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref) - bound))


@torch.no_grad()
def test_deploy_fused_matches_original(bx):
    model = MLP()
    xs = [torch.randn(512, generator=torch.Generator().manual_seed(1)).to(DEV),
          torch.randn(3, 7, 512, generator=torch.Generator().manual_seed(2)).to(DEV)]
    refs = _ref_outputs(model, xs)
    w_up = model.up.weight.data.to(torch.bfloat16)
    b_up = model.up.bias.data
    w_down = model.down.weight.data.to(torch.bfloat16)
    total, n_el = bx.deploy_bf16x_fused(model, verbose=False)
    assert isinstance(model.up, bx.Bf16xFused) and n_el == 2 * 512 * 1536
    for x in xs:
        xb = x.to(torch.bfloat16)
        # bias-free layer: the north-star elementwise tolerance
        h = torch.randn(*x.shape[:-1], 1536, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
        check_tol(model.down(h.to(DEV)).float().cpu().numpy(), h.double().numpy() @ w_down.double().numpy().T)
        # biased layer: the bias is added to the bf16 product in bf16 (bf16x_fused.py:215-216)
        check_biased(model.up(xb), xb.double().cpu().numpy() @ w_up.double().numpy().T, b_up)
    for x, r in zip(xs, refs):
        for mode in ("fused", "opt", "repo"):
            model.up.mode = model.down.mode = mode
            y = model(x.to(torch.bfloat16))
            assert y.shape == x.shape
            assert norm_rel(y.float().cpu().numpy(), r) < 1e-2, mode


@torch.no_grad()
def test_deploy_gemm_saturated_and_exact(bx):
    model = MLP()
    w_up = model.up.weight.data.to(torch.bfloat16)
    x = torch.randn(64, 512, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    # reference numerics: the saturated weight
    d = bx.bf16x_quantize(w_up)
    w_sat = dc.bits_to_f32(dc.decode_saturated({k: (v.numpy() if isinstance(v, torch.Tensor) else v)
                                                for k, v in d.items()}))
    xw_sat = x.double().numpy() @ w_sat.astype(np.float64).T
    xw_exact = x.double().numpy() @ w_up.double().numpy().T
    m_sat = copy.deepcopy(model)
    bx.deploy_bf16x_gemm(m_sat, verbose=False)
    m_ex = copy.deepcopy(model)
    bx.deploy_bf16x_gemm(m_ex, verbose=False, exact=True)
    assert isinstance(m_sat.up, bx.Bf16xGemmLinear) and not m_sat.up.exact and m_ex.up.exact
    check_biased(m_sat.up(x.to(DEV)), xw_sat, model.up.bias.data)
    check_biased(m_ex.up(x.to(DEV)), xw_exact, model.up.bias.data)
    # the saturated weight differs from the exact one on this weight
    assert not np.array_equal(w_sat, w_up.float().numpy())


@torch.no_grad()
def test_bf16x_linear(bx):
    lin = nn.Linear(1536, 256)
    with torch.no_grad():
        lin.weight.mul_(3.0)
    m = bx.BF16XLinear(lin, device=DEV)
    w = lin.weight.data.to(torch.bfloat16)
    assert torch.equal(m.decoded_weight().cpu(), w.float())
    x1 = torch.randn(1536, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    xm = torch.randn(5, 1536, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    for x in (x1, xm):
        xw = x.double().numpy() @ w.double().numpy().T
        check_biased(m(x.to(DEV)), xw, lin.bias.data)
        m.decode_to_bf16()
        check_biased(m(x.to(DEV)), xw, lin.bias.data)
        m.clear_bf16()
