"""Kernel-level seams: the WY stage of KDA and GDN2.

``chunk_kda_bwd_wy_dqkg_fused`` is keyword-compatible with FLA's function of that name as the
reference replaces its kernel (``backends/backward.py:23-25``: ``LocalBetaResidual``, the
residual producer / consumer pair of ``kernels/kda_residual_local_beta.py:8-23``; the NPU
wrapper's signature, ``kernels/kda_residual_npu_onchip.py:683-702``):
``(q, k, v, v_new, g, beta, A, h, do, dh, dv, scale, ...) -> (dq, dk, dv2, db, dg, dA)``.
``dv`` is the state recurrence's output (FLA's dv after ``chunk_gated_delta_rule_bwd_dhu``,
dR here).  dq, dk, dg (before the reverse cumsum) and db are partial gradients that the
matrix intra completes (``backends.intra.chunk_kda_bwd_intra`` with ``beta_complete=True``:
db is already complete on rows with |beta| >= 1e-6, as the reference's residual producer
makes it); dA is the intra's dAkk.  Runs ``fdr_chunk_bwd_wy``.

``chunk_gdn2_bwd_wy_dqkg_fused`` is keyword-compatible with the reference's GDN2 replacement
``gdn2_consumer_fp32.residual`` (``kernels/gdn2_consumer_fp32.py:76-86``, bound at
``backends/backward.py:43-47``):
``(q, k, v, v_new, g, b, w_gate, A, h, do, dh, dv, scale, ...) -> (dq, dk, dv2, db, dw, dg, dA)``.
The reference's producer leaves dq, dk, db, dg to its joint consumer, which runs inside its
intra seam; here they leave this seam as partial gradients (every term but the matrix intra,
dg before the reverse cumsum) and ``backends.intra.chunk_gdn2_bwd_intra`` adds the intra
terms given dAqk and dA (the reference's DM).  dv2 and dw are complete.  Runs
``fdr_gdn2_chunk_bwd_wy``.

Both take a packed batch (``cu_seqlens``, B = 1, sequences starting anywhere; FLA's
``chunk_indices`` is derived from it and checked when given).  No fallback.
"""
from __future__ import annotations

import torch

from .. import ops


def varlen_of(q, cu_seqlens, chunk_indices, what):
    """The ``ops.Varlen`` of a seam's packed batch, or None; checks FLA's chunk_indices [NC, 2]
    against the chunk count the kernels derive from cu_seqlens."""
    if cu_seqlens is None:
        if chunk_indices is not None:
            raise NotImplementedError(f"{what}: chunk_indices without cu_seqlens")
        return None
    if q.shape[0] != 1:
        raise ValueError(f"The batch size is expected to be 1 rather than {q.shape[0]} when using `cu_seqlens`.")
    vl = cu_seqlens if isinstance(cu_seqlens, ops.Varlen) else ops.Varlen(cu_seqlens, q.device)
    if vl.T != q.shape[1]:
        raise ValueError("cu_seqlens must rise from 0 to T")
    if chunk_indices is not None and tuple(chunk_indices.shape) != (vl.NC, 2):
        raise ValueError(f"chunk_indices must be [{vl.NC}, 2] for these cu_seqlens, got {tuple(chunk_indices.shape)}")
    return vl


def _common(what, chunk_size, use_graph):
    if chunk_size != 64:
        raise NotImplementedError(f"{what}: chunk_size must be 64")
    if use_graph:
        raise NotImplementedError(f"{what}: use_graph is not supported")


def _bf(x):
    return x.to(torch.bfloat16).contiguous()


def _f32(x):
    return x.to(torch.float32).contiguous()


def _states(h, dh, state_v_first):
    # FLA's V-first per-chunk states: h is read as it is, dh is given to the kernel K-first
    return _bf(h), _bf(dh.transpose(-1, -2) if state_v_first else dh)


def chunk_kda_bwd_wy_dqkg_fused(q, k, v, v_new, g, beta, A, h, do, dh, dv, scale=None, state_v_first=False,
                                cu_seqlens=None, chunk_size=64, chunk_indices=None, chunk_offsets=None,
                                use_graph=False):
    """-> (dq, dk, dv2, db, dg, dA); q / k may have fewer heads than v (grouped value
    heads: dq / dk come per value head, as FLA's do)."""
    what = "HIP WY seam"
    _common(what, chunk_size, use_graph)
    vl = varlen_of(q, cu_seqlens, chunk_indices, what)
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    h, dh = _states(h, dh, state_v_first)
    out = ops.chunk_bwd_wy(_bf(q), _bf(k), _bf(v), _bf(v_new), _bf(do), _bf(dv), _f32(g), _f32(A), h, dh, scale,
                           beta=_f32(beta), h_v_first=state_v_first, varlen=vl)
    return out["dq"], out["dk"], out["dv"], out["dbeta"], out["dg"], out["dA"]


def chunk_gdn2_bwd_wy_dqkg_fused(q, k, v, v_new, g, b, w_gate, A, h, do, dh, dv, scale=None, cu_seqlens=None,
                                 chunk_size=64, chunk_indices=None, state_v_first=False, use_graph=False):
    """-> (dq, dk, dv2, db, dw, dg, dA): GDN2 with the vector erase gate b and write gate
    w_gate (one q / k head per value head)."""
    what = "HIP GDN2 WY seam"
    _common(what, chunk_size, use_graph)
    vl = varlen_of(q, cu_seqlens, chunk_indices, what)
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    h, dh = _states(h, dh, state_v_first)
    out = ops.chunk_bwd_wy(_bf(q), _bf(k), _bf(v), _bf(v_new), _bf(do), _bf(dv), _f32(g), _f32(A), h, dh, scale,
                           b=_bf(b), w=_bf(w_gate), h_v_first=state_v_first, varlen=vl)
    return out["dq"], out["dk"], out["dv"], out["db"], out["dw"], out["dg"], out["dA"]
