"""KDA's fused gate activation (``use_gate_in_kernel=True``) and its backward.

The reference documents the activation its FLA kernel fuses with the chunk
cumsum (``_compat/kda.py:250-294``; FLA itself is not part of this build):

* ``g = -exp(A_log[h]) * softplus(g_raw + dt_bias[h, k])``               (default)
* ``g = lower_bound * sigmoid(exp(A_log[h]) * (g_raw + dt_bias[h, k]))`` (``lower_bound`` set)
* ``g = lower_bound * sigmoid(g_raw + dt_bias[h, k])``                   (``lower_bound`` set, no A_log)

with ``g_raw`` [B,T,H,K], ``A_log`` [H] and the optional ``dt_bias`` [H*K].  The
backward returns the gradients of ``g_raw``, ``A_log`` and ``dt_bias`` from the
gradient of the activated gate -- the ``dA_log`` / ``ddt_bias`` outputs of the
reference's ``kda_backward`` (``backends/backward.py:63-73``).  Elementwise fp32.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _pre(g_raw, dt_bias):
    H, K = g_raw.shape[2], g_raw.shape[3]
    x = g_raw.float()
    if dt_bias is not None:
        x = x + dt_bias.float().view(H, K)
    return x


def kda_gate(g_raw, A_log=None, dt_bias=None, lower_bound=None):
    """Activated per-token log decay, fp32 [B,T,H,K]."""
    H = g_raw.shape[2]
    x = _pre(g_raw, dt_bias)
    if lower_bound is None:
        if A_log is None:
            raise ValueError("A_log is required when lower_bound is not set")
        return -torch.exp(A_log.float()).view(H, 1) * F.softplus(x)
    z = x if A_log is None else torch.exp(A_log.float()).view(H, 1) * x
    return lower_bound * torch.sigmoid(z)


def kda_gate_bwd(dg, g_raw, A_log=None, dt_bias=None, lower_bound=None):
    """(dg_raw [B,T,H,K], dA_log [H] | None, ddt_bias [H*K] | None) from dg = dL/dg."""
    H, K = g_raw.shape[2], g_raw.shape[3]
    x = _pre(g_raw, dt_bias)
    dg = dg.float()
    dA = None
    if lower_bound is None:
        a = torch.exp(A_log.float()).view(H, 1)
        dx = -dg * a * torch.sigmoid(x)
        dA = (dg * (-a * F.softplus(x))).sum(dim=(0, 1, 3))
    else:
        a = 1.0 if A_log is None else torch.exp(A_log.float()).view(H, 1)
        s = torch.sigmoid(a * x)
        ds = dg * lower_bound * s * (1 - s)
        dx = ds * a
        if A_log is not None:
            dA = (ds * a * x).sum(dim=(0, 1, 3))
    ddt = None if dt_bias is None else dx.sum(dim=(0, 1)).reshape(H * K).to(dt_bias.dtype)
    if dA is not None:
        dA = dA.to(A_log.dtype)
    return dx.to(g_raw.dtype), dA, ddt


class KDAGate(torch.autograd.Function):
    """The activation as an autograd node (forward ``kda_gate``, backward ``kda_gate_bwd``)."""

    @staticmethod
    def forward(ctx, g_raw, A_log, dt_bias, lower_bound):
        ctx.save_for_backward(g_raw, A_log, dt_bias)
        ctx.lower_bound = lower_bound
        return kda_gate(g_raw, A_log, dt_bias, lower_bound)

    @staticmethod
    def backward(ctx, dg):
        g_raw, A_log, dt_bias = ctx.saved_tensors
        dx, dA, ddt = kda_gate_bwd(dg, g_raw, A_log, dt_bias, ctx.lower_bound)
        return dx, dA, ddt, None
