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

On a GPU both directions run as single-pass HIP kernels (``fdr_kda_gate_fwd`` /
``fdr_kda_gate_bwd``: one read of g_raw and dg, one write, dA_log / ddt_bias summed
per token block and then over the blocks); the torch expressions below are the CPU
path and the original backend's.
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


def _native(x, native):
    return x.is_cuda if native is None else native


def _hip_operands(g_raw, A_log, dt_bias, lower_bound):
    from . import _lib
    B, T, H, K = g_raw.shape
    if K != 128:
        raise ValueError("the HIP gate kernels support K = 128")
    if lower_bound is None and A_log is None:
        raise ValueError("A_log is required when lower_bound is not set")
    raw = g_raw if g_raw.dtype in (torch.float32, torch.bfloat16) else g_raw.float()
    raw = raw.contiguous()
    a = None if A_log is None else A_log.float().contiguous()
    dt = None if dt_bias is None else dt_bias.float().contiguous()
    for x, n, shape in ((a, "A_log", (H,)), (dt, "dt_bias", (H * K,))):
        if x is not None and (tuple(x.shape) != shape or x.device != g_raw.device):
            raise ValueError(f"{n}: expected shape {shape} on {g_raw.device}")
    lb = 0.0 if lower_bound is None else float(lower_bound)
    return _lib, raw, a, dt, int(lower_bound is not None), lb, (B, T, H, K)


def _hip_gate(g_raw, A_log, dt_bias, lower_bound):
    _lib, raw, a, dt, has_lb, lb, (B, T, H, K) = _hip_operands(g_raw, A_log, dt_bias, lower_bound)
    g = torch.empty(B, T, H, K, device=g_raw.device, dtype=torch.float32)
    P = _lib.ptr
    st = _lib.load().fdr_kda_gate_fwd(P(raw), int(raw.dtype == torch.bfloat16), P(a), P(dt), has_lb, lb, P(g),
                                      B, T, H, K, _lib.stream_handle(g_raw.device))
    _lib.check(st, "fdr_kda_gate_fwd")
    return g


def _hip_gate_bwd(dg, g_raw, A_log, dt_bias, lower_bound):
    _lib, raw, a, dt, has_lb, lb, (B, T, H, K) = _hip_operands(g_raw, A_log, dt_bias, lower_bound)
    dev = g_raw.device
    dgf = dg.float().contiguous()
    if tuple(dgf.shape) != (B, T, H, K):
        raise ValueError(f"dg: expected shape {(B, T, H, K)}, got {tuple(dgf.shape)}")
    dx = torch.empty(B, T, H, K, device=dev, dtype=raw.dtype)
    dA = torch.empty(H, device=dev, dtype=torch.float32) if A_log is not None else None
    ddt = torch.empty(H * K, device=dev, dtype=torch.float32) if dt_bias is not None else None
    lib = _lib.load()
    ws = torch.empty(max(1, lib.fdr_kda_gate_workspace_bytes(B, T, H, K) // 4), device=dev, dtype=torch.float32)
    P = _lib.ptr
    st = lib.fdr_kda_gate_bwd(P(dgf), P(raw), int(raw.dtype == torch.bfloat16), P(a), P(dt), has_lb, lb, P(dx),
                              P(dA), P(ddt), P(ws), B, T, H, K, _lib.stream_handle(dev))
    _lib.check(st, "fdr_kda_gate_bwd")
    return (dx.to(g_raw.dtype), None if dA is None else dA.to(A_log.dtype),
            None if ddt is None else ddt.to(dt_bias.dtype))


def kda_gate(g_raw, A_log=None, dt_bias=None, lower_bound=None, native=None):
    """Activated per-token log decay, fp32 [B,T,H,K].  ``native`` (default: on a GPU)
    runs the HIP kernel."""
    if _native(g_raw, native):
        return _hip_gate(g_raw, A_log, dt_bias, lower_bound)
    H = g_raw.shape[2]
    x = _pre(g_raw, dt_bias)
    if lower_bound is None:
        if A_log is None:
            raise ValueError("A_log is required when lower_bound is not set")
        return -torch.exp(A_log.float()).view(H, 1) * F.softplus(x)
    z = x if A_log is None else torch.exp(A_log.float()).view(H, 1) * x
    return lower_bound * torch.sigmoid(z)


def kda_gate_bwd(dg, g_raw, A_log=None, dt_bias=None, lower_bound=None, native=None):
    """(dg_raw [B,T,H,K], dA_log [H] | None, ddt_bias [H*K] | None) from dg = dL/dg.
    ``native`` (default: on a GPU) runs the HIP kernel."""
    if _native(g_raw, native):
        return _hip_gate_bwd(dg, g_raw, A_log, dt_bias, lower_bound)
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
    def forward(ctx, g_raw, A_log, dt_bias, lower_bound, native=None):
        ctx.save_for_backward(g_raw, A_log, dt_bias)
        ctx.lower_bound = lower_bound
        ctx.native = native
        return kda_gate(g_raw, A_log, dt_bias, lower_bound, native)

    @staticmethod
    def backward(ctx, dg):
        g_raw, A_log, dt_bias = ctx.saved_tensors
        dx, dA, ddt = kda_gate_bwd(dg, g_raw, A_log, dt_bias, ctx.lower_bound, ctx.native)
        return dx, dA, ddt, None, None


def beta_sigmoid(beta_raw, scale=1.0, native=None):
    """beta = scale * sigmoid(beta_raw), fp32 (``use_beta_sigmoid_in_kernel``; scale 2 with
    ``allow_neg_eigval``).  ``native`` (default: on a GPU) runs ``fdr_beta_sigmoid_fwd``;
    the backward of the native path is folded into the chunk kernel (ops.chunk_bwd's
    ``beta_sigmoid``)."""
    if not _native(beta_raw, native):
        return torch.sigmoid(beta_raw.float()) * scale
    from . import _lib
    x = beta_raw if beta_raw.dtype in (torch.float32, torch.bfloat16) else beta_raw.float()
    x = x.contiguous()
    out = torch.empty(x.shape, device=x.device, dtype=torch.float32)
    if x.numel() == 0:
        return out
    st = _lib.load().fdr_beta_sigmoid_fwd(_lib.ptr(x), int(x.dtype == torch.bfloat16), float(scale), _lib.ptr(out),
                                          x.numel(), _lib.stream_handle(x.device))
    _lib.check(st, "fdr_beta_sigmoid_fwd")
    return out
