"""The original chunked delta-rule backward, as PyTorch ops.

This is the formulation ReWY replaces (FLA's ``chunk_<op>_bwd`` with its
``prepare_wy_repr_bwd`` / ``chunk_kda_bwd_wy_dqkg_fused``): the local WY
backward uses seven matrix products per chunk (the product list of reference
``benchmarks/data/intro_graph_data.json``; readable NPU port of FLA's kernel at
``kernels/gdn_original_separate_npu.py:226-477``)::

    Wb = -dR h^T            T_Z = dR Z^T           Zb = A^T dR
    Eb = A^T Wb             T_E = Wb E^T           J  = A^T (T_Z + T_E)
    D  = -strict_tril(J A^T)

It serves as the ``original`` backend of ``rewy_amd.runtime`` (the role FLA's
unpatched operators play in the reference) and as the same-GPU comparator of
the benchmark.  Shapes and conventions follow ``rewy_amd.forward``.
"""
from __future__ import annotations

import torch

from .forward import from_chunks, recompute, to_chunks, _family_operands, _slices


def _intra(L, D, qf, kf, bk, gcv):
    """Pairwise matrix-intra VJP: (uq, ue, uk) for chunked operands.  gcv is the
    log2 gate ([..,K] vector or [..,1] scalar)."""
    shp = kf.shape
    C, K = shp[-2], shp[-1]
    N = kf.numel() // (C * K)
    L2, D2 = L.reshape(N, C, C), D.reshape(N, C, C)
    q2, k2, bk2 = qf.reshape(N, C, K), kf.reshape(N, C, K), bk.expand(shp).reshape(N, C, K)
    if gcv.shape[-1] == 1:
        g2 = gcv.reshape(N, C)
        low = torch.tril(torch.ones(C, C, dtype=torch.bool, device=kf.device))
        d = g2[:, :, None] - g2[:, None, :]
        f = torch.exp2(torch.where(low, d, torch.full_like(d, -float("inf"))))
        Lf, Df = L2 * f, D2 * f
        uq, ue = Lf @ k2, Df @ k2
        uk = Lf.transpose(1, 2) @ q2 + Df.transpose(1, 2) @ bk2
        return uq.reshape(shp), ue.reshape(shp), uk.reshape(shp)
    g2 = gcv.reshape(N, C, K)
    uq = torch.empty(N, C, K, device=kf.device)
    ue = torch.empty_like(uq)
    uk = torch.empty_like(uq)
    low = torch.tril(torch.ones(C, C, dtype=torch.bool, device=kf.device))
    per = max(1, (1 << 27) // (C * C * K))
    for sl in _slices(N, per):
        d = g2[sl, :, None, :] - g2[sl, None, :, :]
        f = torch.exp2(torch.where(low[None, :, :, None], d, torch.full_like(d, -float("inf"))))
        uq[sl] = torch.einsum("nij,nijk,njk->nik", L2[sl], f, k2[sl])
        ue[sl] = torch.einsum("nij,nijk,njk->nik", D2[sl], f, k2[sl])
        uk[sl] = (torch.einsum("nji,njik,njk->nik", L2[sl], f, q2[sl])
                  + torch.einsum("nji,njik,njk->nik", D2[sl], f, bk2[sl]))
        del d, f
    return uq.reshape(shp), ue.reshape(shp), uk.reshape(shp)


def original_backward(op, q, k, v, gc, Akk, scale, initial_state, do, dht, beta=None, b=None,
                      w=None, Aqk=None, saved=None):
    """Full backward in the original (7-product) formulation.

    Returns dict(dq, dk, dv, dg (raw gate, gate shape) | None, dbeta | None,
    db, dw | None, dh0 | None) in fp32."""
    B, T, H, K = q.shape
    dev = q.device
    qf, kf, vf, gcv, bc, wc = _family_operands(op, q, k, v, gc, beta, b, w)
    if saved is None or saved.get("h") is None:
        saved = recompute(op, q, k, v, gc, Akk, beta=beta, b=b, w=w, initial_state=initial_state)
    A = to_chunks(Akk.float())
    NT = T // 64
    if Aqk is None:
        from .backends.backward import _aqk_scalar
        Aqk = _aqk_scalar(q, k, gc, scale)
    Aq = to_chunks(Aqk.float())
    R = to_chunks(saved["v_new"].float())
    hs = saved["h"].float().permute(0, 2, 1, 3, 4)                    # [B,H,NT,K,V]
    wwy = to_chunks(saved["w"].float())
    qg = to_chunks(saved["qg"].float())
    kg = to_chunks(saved["kg"].float())
    dOc = to_chunks(do.float())
    gam = torch.exp2(gcv)
    lam = torch.exp2(gcv[..., -1, :])                                  # [B,H,NT,K|1]
    # dAv: dAqk and dv_local (FLA chunk_kda_bwd_dAv / chunk_bwd_dv_local)
    low = torch.tril(torch.ones(64, 64, dtype=torch.bool, device=dev))
    L = torch.where(low, scale * (dOc @ R.transpose(-1, -2)), torch.zeros((), device=dev))
    dvl = Aq.transpose(-1, -2) @ dOc
    # reverse state recurrence (FLA chunk_gated_delta_rule_bwd_dhu)
    dh = torch.empty_like(hs)
    dR = torch.empty_like(R)
    st = torch.zeros(B, H, K, v.shape[-1], device=dev) if dht is None else dht.float().clone()
    for c in reversed(range(NT)):
        dh[:, :, c] = st.to(torch.bfloat16).float()
        dR[:, :, c] = kg[:, :, c] @ dh[:, :, c] + dvl[:, :, c]
        st = (lam[:, :, c, :, None] * st + scale * qg[:, :, c].transpose(-1, -2) @ dOc[:, :, c]
              - wwy[:, :, c].transpose(-1, -2) @ dR[:, :, c])
    dh0 = st if initial_state is not None else None
    # original WY backward: seven products
    E = bc * kf * gam
    Z = wc * vf
    At = A.transpose(-1, -2)
    Wb = -(dR @ hs.transpose(-1, -2))                                  # 1
    TZ = dR @ Z.transpose(-1, -2)                                      # 2
    Zb = At @ dR                                                       # 3
    Eb = At @ Wb                                                       # 4
    TE = Wb @ E.transpose(-1, -2)                                      # 5
    J = At @ (TZ + TE)                                                 # 6
    D = -torch.tril(J @ At, -1)                                        # 7
    # state-gradient terms
    dq_s = (dOc @ hs.transpose(-1, -2)) * gam * scale
    dks = (R @ dh.transpose(-1, -2)) * torch.exp2(gcv[..., -1:, :] - gcv)
    uq, ue, uk = _intra(L, D, qf, kf, bc * kf, gcv)
    dq = dq_s + uq
    dk = dks + bc * gam * Eb + bc * ue + uk
    dv = wc * Zb
    dbv = kf * gam * Eb + kf * ue                                      # grad of b (per K)
    dwv = vf * Zb                                                      # grad of w (per V)
    dG = qf * dq - kf * dks + bc * kf * gam * Eb + kf * (bc * ue - uk)
    dG[..., -1, :] += lam * (hs * dh).sum(-1) + (kf * dks).sum(-2)
    dg = dG.flip(-2).cumsum(-2).flip(-2)
    out = dict(dq=from_chunks(dq), dk=from_chunks(dk), dv=from_chunks(dv), dh0=dh0,
               dg=None, dbeta=None, db=None, dw=None)
    if op == "gdn2":
        out["db"], out["dw"] = from_chunks(dbv), from_chunks(dwv)
    else:
        out["dbeta"] = from_chunks(dbv.sum(-1, keepdim=True) + dwv.sum(-1, keepdim=True))[..., 0]
    if op in ("kda", "gdn2"):
        out["dg"] = from_chunks(dg)
    elif op == "gdn":
        out["dg"] = from_chunks(dg.sum(-1, keepdim=True))[..., 0]
    return out
