"""Kernel-level seam: the matrix intra of the vector-gated families.

Keyword-compatible with FLA's ``chunk_kda_bwd_intra`` / ``chunk_gdn2_bwd_intra``
as the reference replaces them (``backends/backward.py:18-25,44-49``):
``(q, k, g, beta|b, dAqk, dAkk, dq, dk, db, dg, ...) -> (dq, dk, db, dg)``, with
dq, dk, db, dg fp32 partial gradients updated in place (the reference's
``EndpointMatrixIntra.__call__``, ``kernels/endpoint_intra.py:300-326``, writes
``dq2`` over ``dq``).  Runs ``fdr_matrix_intra``; no fallback.
"""
from __future__ import annotations

import torch

from .. import ops


def _check(kw, chunk_size):
    for name in ("cu_seqlens", "chunk_indices"):
        if kw.get(name) is not None:
            raise NotImplementedError(f"HIP matrix intra: {name} is not supported")
    if chunk_size != 64:
        raise NotImplementedError("HIP matrix intra: chunk_size must be 64")
    if kw.get("safe_gate", False) or kw.get("use_graph", False):
        raise NotImplementedError("HIP matrix intra: safe_gate / use_graph are not supported")


def _prep(q, k, g, dAqk, dAkk):
    return (q.to(torch.bfloat16).contiguous(), k.to(torch.bfloat16).contiguous(),
            g.to(torch.float32).contiguous(), dAqk.to(torch.float32).contiguous(),
            dAkk.to(torch.float32).contiguous())


def chunk_kda_bwd_intra(q, k, g, beta, dAqk, dAkk, dq, dk, db, dg, cu_seqlens=None, chunk_indices=None,
                        chunk_size=64, safe_gate=False, lower_bound=None, use_graph=False, beta_complete=False):
    """KDA intra: db += sum_k ue k on every row (FLA semantics), or only on rows with
    |beta| < 1e-6 when ``beta_complete`` (ReWY's residual path, ``endpoint_intra.py:190-194``)."""
    _check(dict(cu_seqlens=cu_seqlens, chunk_indices=chunk_indices, safe_gate=safe_gate, use_graph=use_graph),
           chunk_size)
    q, k, g, dAqk, dAkk = _prep(q, k, g, dAqk, dAkk)
    return ops.matrix_intra(q, k, g, dAqk, dAkk, dq, dk, db, dg, beta=beta.to(torch.float32).contiguous(),
                            beta_complete=beta_complete)


def chunk_gdn2_bwd_intra(q, k, g, b, dAqk, dAkk, dq, dk, db, dg, cu_seqlens=None, chunk_indices=None,
                         chunk_size=64, **unused):
    """GDN2 intra with the vector erase gate b: db += ue k elementwise."""
    _check(dict(cu_seqlens=cu_seqlens, chunk_indices=chunk_indices, **unused), chunk_size)
    q, k, g, dAqk, dAkk = _prep(q, k, g, dAqk, dAkk)
    return ops.matrix_intra(q, k, g, dAqk, dAkk, dq, dk, db, dg, b=b.to(torch.bfloat16).contiguous())
