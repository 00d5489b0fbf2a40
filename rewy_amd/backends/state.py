"""Kernel-level seam: the reverse inter-chunk state recurrence.

Keyword-compatible with FLA's ``chunk_gated_delta_rule_bwd_dhu`` as the reference replaces
it for GDN2 (``kernels/vector_state_gpu.py:47-67``, ``state_bwd``, bound at
``backends/backward.py:43-47``) and as FLA calls it for KDA, GDN and DeltaNet
(``backends/backward.py:120-121``):
``(q, k, w, do, dv, g=None, gk=None, h0=None, dht=None, scale=None, state_v_first=False,
cu_seqlens=None, ...) -> (dh, dh0, dr)``.

Per (sequence, head), from dht (or zero) over the chunks in reverse:
``dh[c] = dh; dr_c = dv_c + k_c dh; dh = lambda_c dh + scale q_c^T dO_c - w_c^T dr_c``, with the
vector gate ``gk`` (k, q given gate-weighted, kg and qg, as FLA's KDA / GDN2 pass them), the
scalar gate ``g`` (raw q, k; the kernel applies 2^(g_last - g_t) to k and 2^g_t to q), or none
(DeltaNet).  Gates are chunk-local cumsums in log2 units.  dh is [B, NT, HV, K, V] in q's dtype
(bf16; [.., V, K] under ``state_v_first``, as are dht and dh0), dh0 fp32 when h0 is given, dr
has dv's shape.  ``value_block`` is the reference's Triton tile width; the kernel picks its own
tiles (the results do not depend on them).  Runs ``fdr_state_bwd`` (or, with ``cu_seqlens``,
``fdr_state_bwd_varlen``).  No fallback.
"""
from __future__ import annotations

import torch

from .. import ops
from .wy import varlen_of


def chunk_gated_delta_rule_bwd_dhu(q, k, w, do, dv, g=None, gk=None, h0=None, dht=None, scale=None,
                                   state_v_first=False, cu_seqlens=None, chunk_size=64, chunk_indices=None,
                                   chunk_offsets=None, value_block=16, use_exp2=True, **unused):
    """-> (dh, dh0, dr).  q / k may have fewer heads than w / do / dv (grouped value heads)."""
    if chunk_size != 64:
        raise NotImplementedError("HIP state recurrence: chunk_size must be 64")
    if not use_exp2:
        raise NotImplementedError("HIP state recurrence: gates are log2-unit cumsums (use_exp2=True)")
    if g is not None and gk is not None:
        raise ValueError("pass at most one of g (scalar gate) / gk (vector gate)")
    vl = varlen_of(q, cu_seqlens, chunk_indices, "HIP state recurrence")
    if vl is not None and chunk_offsets is not None and chunk_offsets.numel() != vl.N + 1:
        raise ValueError(f"chunk_offsets must hold {vl.N + 1} entries for these cu_seqlens")
    bf, f32 = torch.bfloat16, torch.float32
    if gk is not None:
        gate, gg = ops.GATE_VECTOR, gk.to(f32).contiguous()
    elif g is not None:
        gate, gg = ops.GATE_SCALAR, g.to(f32).contiguous()
    else:
        gate, gg = ops.GATE_NONE, None
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    c = lambda x: x.to(bf).contiguous()
    dh, dr, dh0 = ops.state_bwd(c(q), c(k), c(w), gg, gate, c(do), scale, dv=c(dv),
                                dht=None if dht is None else dht.to(f32).contiguous(), want_dh0=h0 is not None,
                                state_v_first=state_v_first, varlen=vl)
    if state_v_first:
        dh = dh.transpose(-1, -2).contiguous()
    return dh.to(q.dtype), dh0, dr.to(dv.dtype)
