"""GPU tests of the bf16x-v1 loader: a model re-loaded from disk decodes
every packed weight bit-exactly and gives the original model's outputs, in
both modes (fused kernels; decode then F.linear)."""
import copy

import numpy as np
import pytest
import torch

from tests.test_disk_host import Tiny
from tests.test_gpu_dict import DEV, check_tol
from tests.test_gpu_modules import check_biased

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def bx():
    import bfloat16x_amd as m
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return m


@torch.no_grad()
def test_reload_from_disk(bx, tmp_path):
    from bfloat16x_amd import disk
    model = Tiny()
    orig = copy.deepcopy(model)
    prefix = str(tmp_path / "tiny")
    disk.pack_model_to_disk(model, prefix, verbose=False)
    fresh = Tiny()                                    # same architecture, weights to be replaced
    n = disk.replace_linears_from_packed(fresh, prefix, verbose=False, device=DEV)
    assert n == 2 and isinstance(fresh.up, disk.Bf16xStreamLinear) and isinstance(fresh.down, disk.Bf16xStreamLinear)
    assert fresh.small.weight.dtype == torch.bfloat16 and fresh.small.weight.is_cuda
    for nm in ("up", "down"):
        w = getattr(orig, nm).weight.data.to(torch.bfloat16)
        assert torch.equal(getattr(fresh, nm).decoded_weight().cpu().view(torch.int16), w.view(torch.int16))
    x1 = torch.randn(64, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    xm = torch.randn(5, 64, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    wu = orig.up.weight.data.to(torch.bfloat16).double().numpy()
    wd = orig.down.weight.data.to(torch.bfloat16).double().numpy()
    for mode in ("fused", "decode"):
        fresh.up.mode = fresh.down.mode = mode
        for x in (x1, xm):
            check_biased(fresh.up(x.to(DEV)), x.double().numpy() @ wu.T, orig.up.bias.data)
            h = torch.randn(*x.shape[:-1], 192, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
            check_tol(fresh.down(h.to(DEV)).float().cpu().numpy(), h.double().numpy() @ wd.T)
