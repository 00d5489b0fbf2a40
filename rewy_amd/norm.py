"""q / k L2 normalisation over the key dimension (``use_qk_l2norm_in_kernel=True``,
reference ``_compat/kda.py:202-206``; FLA's ``l2norm_fwd`` / ``l2norm_bwd``):
``y = x / sqrt(sum_k x^2 + eps)``, eps = 1e-6, computed in fp32 and returned in x's dtype.

On a GPU (the optimized backend) forward and backward are single-pass HIP kernels
(``fdr_l2norm_fwd`` saves the fp32 reciprocal norm per row, ``fdr_l2norm_bwd`` forms
``dx = r (dy - y (y . dy))`` from x, r and dy); elsewhere the torch expression runs
under autograd.
"""
from __future__ import annotations

import torch

EPS = 1e-6


def l2norm_torch(x, eps=EPS):
    xf = x.float()
    return (xf * torch.rsqrt((xf * xf).sum(-1, keepdim=True) + eps)).to(x.dtype)


def _check(x):
    if x.shape[-1] != 128:
        raise ValueError("the HIP l2norm kernels support a last dimension of 128")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"l2norm: bf16 or fp32 expected, got {x.dtype}")


class L2Norm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        from . import _lib
        _check(x)
        x = x.contiguous()
        rows = x.numel() // 128
        y = torch.empty_like(x)
        rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
        P = _lib.ptr
        st = _lib.load().fdr_l2norm_fwd(P(x), int(x.dtype == torch.bfloat16), P(y), P(rstd), rows, 128, EPS,
                                        _lib.stream_handle(x.device))
        _lib.check(st, "fdr_l2norm_fwd")
        ctx.save_for_backward(x, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        from . import _lib
        x, rstd = ctx.saved_tensors
        dy = dy.to(x.dtype).contiguous()
        dx = torch.empty_like(x)
        P = _lib.ptr
        st = _lib.load().fdr_l2norm_bwd(P(x), int(x.dtype == torch.bfloat16), P(rstd), P(dy), P(dx),
                                        x.numel() // 128, 128, _lib.stream_handle(x.device))
        _lib.check(st, "fdr_l2norm_bwd")
        return dx


def l2norm(x, native=None):
    """L2-normalised x (autograd-aware); ``native`` (default: on a GPU) uses the HIP kernels."""
    if x.is_cuda if native is None else native:
        return L2Norm.apply(x)
    return l2norm_torch(x)
