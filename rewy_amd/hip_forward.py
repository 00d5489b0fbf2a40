"""The chunked forward on the gfx950 kernels (the optimized backend's forward).

Stands where the reference calls FLA's ``chunk_kda_fwd`` / ``chunk_gdn2_fwd`` /
``chunk_gated_delta_rule_fwd`` / ``chunk_delta_rule_fwd`` (reference
``_compat/kda.py:89-113``, ``_compat/gdn.py:33-123``, ``_compat/gdn2.py:87-108``)
and returns the same (o, final_state, saved) as ``rewy_amd.forward.chunk_forward``
(its PyTorch restatement, used by the original backend and on the CPU):

  1. ``fdr_fwd_prepare`` -- gc (log2 chunk-local cumsum), Aqk, Akk = (I + M)^-1;
  2. ``fdr_prepare_wu``  -- w, u (and qg, kg for vector gates);
  3. ``fdr_fwd_h``       -- per-chunk states h, v_new and the final state
     (2-3 as one sweep, ``fdr_fwd_h_wy``, where that pays);
  4. ``fdr_fwd_o``       -- o = scale (q 2^gc) h + Aqk v_new.

No fallback: a missing HIP library raises.
"""
from __future__ import annotations

import torch

from . import ops

GATE_MODE = {"delta": ops.GATE_NONE, "gdn": ops.GATE_SCALAR, "kda": ops.GATE_VECTOR, "gdn2": ops.GATE_VECTOR}


def chunk_forward_hip(op, q, k, v, g=None, beta=None, b=None, w=None, initial_state=None, scale=None,
                      output_final_state=False, varlen=None, state_v_first=False, fuse_scan=None):
    """``varlen`` (an ``ops.Varlen``): B = 1 holds sequences packed along T, starting
    anywhere (FLA's cu_seqlens); initial / final states are per sequence, and every stage
    takes the batch's chunk map (a sequence's last chunk may be partial).  ``state_v_first``:
    initial / final states are [N,H,V,K] (read and written so by ``fwd_h``); the saved
    per-chunk h stays [B,NT,H,K,V].  ``fuse_scan``: steps 2-3 as one sweep (``fdr_fwd_h_wy``,
    the same bits, u not materialized: saved ``u`` is None) -- by default where that pays
    (``ops.fwd_h_wy_pays``)."""
    B, T, H, K = q.shape
    scale = K ** -0.5 if scale is None else scale
    gm = GATE_MODE[op]
    bf, f32 = torch.bfloat16, torch.float32
    q, k, v = (x.to(bf).contiguous() for x in (q, k, v))
    g = None if gm == ops.GATE_NONE else g.to(f32).contiguous()
    vb = op == "gdn2"
    beta = None if vb else beta.to(f32).contiguous()
    b = b.to(bf).contiguous() if vb else None
    w = w.to(bf).contiguous() if vb else None
    h0 = None if initial_state is None else initial_state.to(f32).contiguous()
    gc, Aqk, Akk = ops.fwd_prepare(q, k, g, gm, beta=beta, b=b, scale=scale, varlen=varlen)
    vec = gm == ops.GATE_VECTOR
    N, H = (B if varlen is None else varlen.N), v.shape[2]
    if fuse_scan is None:
        fuse_scan = not ops._use_affine("auto", N, H, T // ops.CHUNK) and ops.fwd_h_wy_pays(N, H, gm, varlen)
    if fuse_scan:
        wu = ops.fwd_h_wy(k, v, Akk, gc, gm, beta=beta, q=q if vec else None, b=b, w=w, h0=h0,
                          want_final=output_final_state, varlen=varlen, state_v_first=state_v_first)
        wu["u"] = None
        h, v_new, final = wu["h"], wu["v_new"], wu["final"]
    else:
        wu = ops.prepare_wu(k, v, Akk, gm, g=gc, beta=beta, b=b, w=w, q=q, want_qkg=vec, scale=scale,
                            varlen=varlen)
        h, v_new, final = ops.fwd_h(wu["kg"] if vec else k, wu["w"], wu["u"], gc, gm, h0=h0,
                                    want_final=output_final_state, varlen=varlen,
                                    method="auto" if varlen is None else "direct", state_v_first=state_v_first)
    o = ops.fwd_o(q, gc, gm, Aqk, h, v_new, scale, varlen=varlen)
    saved = dict(gc=gc, Aqk=Aqk, Akk=Akk, w=wu["w"], u=wu["u"], qg=wu["qg"], kg=wu["kg"], v_new=v_new, h=h,
                 scale=scale)
    return o, final, saved
