"""Configurations 2 and 3 at their stated sizes, on the benchmark's own
weights (bench.bench_weight: torch generator, N(0, 0.02), 1 % x30, seed 0):
the exact decode returns the original bits, the fused GEMV at every
configuration-2 shape and the fused / default decode+GEMM at the
configuration-3 shapes match an fp64 product of the original weight within
the north-star tolerance (max 1e-2, median 2e-3).  Reference shapes:
bf16x_fused.py:114-127 (GEMV), bf16x_gemm_fused.py:97-114 (GEMM)."""
import pytest
import torch

from bench import bench_weight
from tests.test_gpu_dict import DEV, check_tol

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def bx():
    import bfloat16x_amd as m
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return m


_W = {}


def _weight(bx, out_f, in_f):
    """(bf16 weight on the device, streams, plan) for one shape, built once."""
    key = (out_f, in_f)
    if key not in _W:
        _W.clear()
        torch.cuda.empty_cache()
        wd = bench_weight(out_f, in_f, seed=0).to(DEV)
        d = bx.bf16x_quantize(wd)                                  # device encoder
        plan = bx.build_plan_host(d, device=DEV)
        streams = (d["sign_packed"], d["mant_packed"], d["delta_packed"], d["emax"])
        dec = bx.bf16x_decode(*streams, out_f, in_f, plan=plan)
        assert torch.equal(dec.view(torch.int16), wd.view(torch.int16)), "exact decode != original bits"
        _W[key] = (wd, streams, plan)
    return _W[key]


@pytest.mark.parametrize("shape", [(4096, 4096), (1024, 4096), (4096, 14336)])
def test_config2_gemv_full_size(bx, shape):
    out_f, in_f = shape
    print("config2 gemv full size", shape, flush=True)
    wd, streams, plan = _weight(bx, out_f, in_f)
    x = torch.randn(in_f, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(DEV)
    y = bx.bf16x_gemv(x, *streams, out_f, in_f, plan=plan)
    y_ref = (wd.double() @ x.double()).cpu().numpy()
    mx, med = check_tol(y.float().cpu().numpy(), y_ref)
    print(f"  rel err max {mx:.2e} median {med:.2e}", flush=True)


@pytest.mark.parametrize("shape,M", [((4096, 4096), 256), ((4096, 4096), 2048), ((4096, 14336), 2048),
                                     ((14336, 4096), 2048), ((4096, 14336), 256), ((4096, 4096), 16),
                                     ((4096, 14336), 64)])
def test_config3_gemm_full_size(bx, shape, M):
    out_f, in_f = shape
    print("config3 gemm full size", shape, "M", M, flush=True)
    wd, streams, plan = _weight(bx, out_f, in_f)
    x = torch.randn(M, in_f, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16).to(DEV)
    y_ref = (x.double() @ wd.double().t().contiguous()).cpu().numpy()
    for path in ("fused", "auto"):
        y = bx.bf16x_gemm(x, *streams, out_f, in_f, plan=plan, path=path)
        assert y.shape == (M, out_f) and y.dtype == torch.bfloat16
        mx, med = check_tol(y.float().cpu().numpy(), y_ref)
        print(f"  {path}: rel err max {mx:.2e} median {med:.2e}", flush=True)
