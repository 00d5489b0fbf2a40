"""Kernel-level seam: the matrix intra of the vector-gated families.

Keyword-compatible with FLA's ``chunk_kda_bwd_intra`` / ``chunk_gdn2_bwd_intra``
as the reference replaces them (``backends/backward.py:18-25,44-49``):
``(q, k, g, beta|b, dAqk, dAkk, dq, dk, db, dg, ...) -> (dq, dk, db, dg)``, with
dq, dk, db, dg fp32 partial gradients updated in place (the reference's
``EndpointMatrixIntra.__call__``, ``kernels/endpoint_intra.py:300-326``, writes
``dq2`` over ``dq``).  A packed batch (``cu_seqlens``, B = 1, sequences starting anywhere;
``endpoint_intra.py:318-321``, ``gdn2_consumer_fp32.py:91-94``) runs
``fdr_matrix_intra_varlen``; dense rows ``fdr_matrix_intra``.  No fallback.
"""
from __future__ import annotations

import torch

from .. import ops
from .wy import varlen_of


def _check(kw, chunk_size):
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
    _check(dict(safe_gate=safe_gate, use_graph=use_graph), chunk_size)
    vl = varlen_of(q, cu_seqlens, chunk_indices, "HIP matrix intra")
    q, k, g, dAqk, dAkk = _prep(q, k, g, dAqk, dAkk)
    return ops.matrix_intra(q, k, g, dAqk, dAkk, dq, dk, db, dg, beta=beta.to(torch.float32).contiguous(),
                            beta_complete=beta_complete, varlen=vl)


def chunk_gdn2_bwd_intra(q, k, g, b, dAqk, dAkk, dq, dk, db, dg, cu_seqlens=None, chunk_indices=None,
                         chunk_size=64, **unused):
    """GDN2 intra with the vector erase gate b: db += ue k elementwise."""
    _check(unused, chunk_size)
    vl = varlen_of(q, cu_seqlens, chunk_indices, "HIP matrix intra")
    q, k, g, dAqk, dAkk = _prep(q, k, g, dAqk, dAkk)
    return ops.matrix_intra(q, k, g, dAqk, dAkk, dq, dk, db, dg, b=b.to(torch.bfloat16).contiguous(), varlen=vl)
