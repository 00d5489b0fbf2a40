"""Kernel-level seam: KDA's WY stage.

Keyword-compatible with FLA's ``chunk_kda_bwd_wy_dqkg_fused`` as the reference replaces
its kernel (``backends/backward.py:23-25``: ``LocalBetaResidual``, the residual producer /
consumer pair of ``kernels/kda_residual_local_beta.py:8-23``; the NPU wrapper's signature,
``kernels/kda_residual_npu_onchip.py:683-702``):
``(q, k, v, v_new, g, beta, A, h, do, dh, dv, scale, ...) -> (dq, dk, dv2, db, dg, dA)``.
``dv`` is the state recurrence's output (FLA's dv after ``chunk_gated_delta_rule_bwd_dhu``,
dR here).  dq, dk, dg (before the reverse cumsum) and db are partial gradients that the
matrix intra completes (``backends.intra.chunk_kda_bwd_intra`` with ``beta_complete=True``:
db is already complete on rows with |beta| >= 1e-6, as the reference's residual producer
makes it); dA is the intra's dAkk.  Runs ``fdr_chunk_bwd_wy``; no fallback.
"""
from __future__ import annotations

import torch

from .. import ops


def chunk_kda_bwd_wy_dqkg_fused(q, k, v, v_new, g, beta, A, h, do, dh, dv, scale=None, state_v_first=False,
                                cu_seqlens=None, chunk_size=64, chunk_indices=None, chunk_offsets=None,
                                use_graph=False):
    """-> (dq, dk, dv2, db, dg, dA); q / k may have fewer heads than v (grouped value
    heads: dq / dk come per value head, as FLA's do)."""
    if cu_seqlens is not None or chunk_indices is not None or chunk_offsets is not None:
        raise NotImplementedError("HIP WY seam: packed cu_seqlens batches run through kda_backward")
    if chunk_size != 64:
        raise NotImplementedError("HIP WY seam: chunk_size must be 64")
    if use_graph:
        raise NotImplementedError("HIP WY seam: use_graph is not supported")
    bf = torch.bfloat16
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    if state_v_first:
        # FLA's V-first per-chunk states: h is read as it is, dh is given to the kernel K-first
        dh = dh.transpose(-1, -2)
    out = ops.chunk_bwd_wy(q.to(bf).contiguous(), k.to(bf).contiguous(), v.to(bf).contiguous(),
                           v_new.to(bf).contiguous(), do.to(bf).contiguous(), dv.to(bf).contiguous(),
                           g.to(torch.float32).contiguous(), A.to(torch.float32).contiguous(), h.to(bf).contiguous(),
                           dh.to(bf).contiguous(), scale, beta.to(torch.float32).contiguous(),
                           h_v_first=state_v_first)
    return out["dq"], out["dk"], out["dv"], out["dbeta"], out["dg"], out["dA"]
