"""HIP q/k L2 normalisation (fdr_l2norm_fwd / _bwd) against torch autograd of the same
expression (y = x / sqrt(sum x^2 + 1e-6), fp32 inside).  fp32: rel-L2 <= 1e-6;
bf16 outputs: <= 4e-3 (one bf16 rounding each side)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _rel(a, r):
    a, r = a.detach().double().cpu(), r.detach().double().cpu()
    return float((a - r).norm() / r.norm().clamp_min(1e-30))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 192, 3), (1, 1000, 5), (1, 1, 1)])
def test_hip_l2norm_matches_torch(dtype, shape):
    from rewy_amd.norm import l2norm, l2norm_torch
    print(f"\n[l2norm] dtype={dtype} shape={shape}", flush=True)
    gen = torch.Generator().manual_seed(5)
    x = (torch.randn(*shape, 128, generator=gen) * 2).to(dtype).cuda()
    dy = torch.randn(*shape, 128, generator=gen).to(dtype).cuda()
    xa = x.clone().requires_grad_()
    xb = x.clone().requires_grad_()
    ya = l2norm(xa, native=True)
    yb = l2norm_torch(xb)
    (ga,) = torch.autograd.grad(ya, xa, dy)
    (gb,) = torch.autograd.grad(yb, xb, dy)
    torch.cuda.synchronize()
    tol = 1e-6 if dtype == torch.float32 else 4e-3
    assert ya.dtype == dtype and ga.dtype == dtype
    assert _rel(ya, yb) < tol, _rel(ya, yb)
    assert _rel(ga, gb) < (1e-5 if dtype == torch.float32 else 1e-2), _rel(ga, gb)
