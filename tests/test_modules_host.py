"""CPU tests of the drop-in modules' surgery (no kernel runs): which layers
deploy_* replaces, the reference's byte accounting, and that the modules
refuse CPU inputs (there is no CPU path)."""
import pytest
import torch
from torch import nn

import bfloat16x_amd as bx
from bfloat16x_amd.nn import packed_bytes


class Toy(nn.Module):
    def __init__(self):
        super().__init__()
        g = torch.Generator().manual_seed(0)
        self.embed_tokens = nn.Linear(64, 64)
        self.block = nn.ModuleDict({"up": nn.Linear(64, 128), "down": nn.Linear(128, 64, bias=False),
                                    "tiny": nn.Linear(16, 16)})
        self.lm_head = nn.Linear(64, 96)
        for p in self.parameters():
            p.data = torch.randn(p.shape, generator=g) * 0.05


@pytest.mark.parametrize("deploy", ["fused", "gemm"])
def test_deploy_selects_layers_and_accounts_like_reference(deploy):
    m = Toy()
    up_w = m.block["up"].weight.data.to(torch.bfloat16).clone()
    if deploy == "fused":
        total, n_el = bx.deploy_bf16x_fused(m, verbose=False, device="cpu")
        cls = bx.Bf16xFused
    else:
        total, n_el = bx.deploy_bf16x_gemm(m, verbose=False, device="cpu")
        cls = bx.Bf16xGemmLinear
    assert isinstance(m.block["up"], cls) and isinstance(m.block["down"], cls)
    assert isinstance(m.block["tiny"], nn.Linear)                   # 256 < 1000 weights
    assert isinstance(m.lm_head, nn.Linear) and isinstance(m.embed_tokens, nn.Linear)
    assert n_el == 64 * 128 * 2
    assert total >= packed_bytes(bx.bf16x_quantize(up_w))
    with pytest.raises(ValueError):                                 # no CPU path
        m.block["up"](torch.randn(64))


def test_gemm_linear_refuses_streaming_mode():
    p = bx.bf16x_quantize(torch.randn(8, 64))
    with pytest.raises(NotImplementedError):
        bx.Bf16xGemmLinear(p, resident=False, device="cpu")


def test_bf16x_linear_from_packed_buffers():
    lin = nn.Linear(64, 32)
    b = bx.bf16x_quantize(lin.weight.data)
    m = bx.BF16XLinear.from_packed(b, bias=lin.bias.data, device="cpu")
    assert m.out_f == 32 and m.in_f == 64 and m.weight.shape == (1, 1)
    assert set(dict(m.named_buffers())) >= {"emax", "sign_packed", "mant_packed", "delta_packed",
                                            "delta_ovf_idx", "delta_ovf_val"}
    with pytest.raises(ValueError):
        m(torch.randn(64))
