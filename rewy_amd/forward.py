"""Chunked delta-rule forward (PyTorch ops) producing the intermediates the
backward consumes, for DeltaNet, GDN, KDA and GDN2.

The forward is not the hot path of this package: it stands where the
reference calls FLA's ``chunk_kda_fwd`` / ``chunk_gated_delta_rule_fwd`` /
``chunk_gdn2_fwd`` / ``chunk_delta_rule_fwd`` (reference
``_compat/kda.py:89-113``, ``_compat/gdn.py:33-123``, ``_compat/gdn2.py:87-108``)
and returns the same set of saved tensors in FLA's layouts:

* ``gc``   fp32 chunk-local cumsum of the gate in log2 units
  (``chunk_local_cumsum(g, scale=RCP_LN2)``, reference ``_compat/gdn.py:63-69``);
* ``Aqk``  fp32 ``[B,T,H,64]``  scale * tril(q k^T * 2^(g_i-g_j)) per chunk;
* ``Akk``  fp32 ``[B,T,H,64]``  (I + strict_tril(b k k^T * 2^(g_i-g_j)))^-1;
* ``w, u`` bf16 WY factors  w = Akk (b k 2^g), u = Akk (w_gate v);
* ``qg, kg`` bf16  q 2^g, k 2^(g_last - g);
* ``v_new`` bf16 ``u - w h``; ``h`` bf16 ``[B,NT,H,K,V]`` state at each chunk start.

Everything is computed in fp32 with pairwise gate factors (never 2^-g
alone), so any gate span stays finite.
"""
from __future__ import annotations

import math

import torch

RCP_LN2 = 1.0 / math.log(2.0)
CHUNK = 64


def to_chunks(x: torch.Tensor, C: int = CHUNK) -> torch.Tensor:
    """[B,T,H,*] -> [B,H,NT,C,*]"""
    B, T, H = x.shape[:3]
    y = x.reshape(B, T // C, C, H, *x.shape[3:])
    perm = (0, 3, 1, 2) + tuple(range(4, y.ndim))
    return y.permute(*perm)


def from_chunks(x: torch.Tensor) -> torch.Tensor:
    """[B,H,NT,C,*] -> [B,T,H,*] (contiguous)"""
    B, H, NT, C = x.shape[:4]
    perm = (0, 2, 3, 1) + tuple(range(4, x.ndim))
    return x.permute(*perm).reshape(B, NT * C, H, *x.shape[4:]).contiguous()


def chunk_local_cumsum(g: torch.Tensor, C: int = CHUNK, scale: float = RCP_LN2) -> torch.Tensor:
    """Per-chunk inclusive cumsum along T, times ``scale`` (fp32)."""
    B, T = g.shape[:2]
    y = g.float().reshape(B, T // C, C, *g.shape[2:]).cumsum(2) * scale
    return y.reshape(g.shape)


def _slices(n: int, per: int):
    for s in range(0, n, per):
        yield slice(s, min(n, s + per))


def _pair_products(q, k, bk, gcv, scale, want_qk=True):
    """Pairwise-gated chunk matrices for vector gates.

    q, k, bk: [N,C,K] fp32, gcv: [N,C,K] log2 cumsum.  Returns
    Aqk = scale * sum_k q_ik k_jk 2^(g_ik-g_jk) (j <= i) and
    Mkk = sum_k bk_ik k_jk 2^(g_ik-g_jk) (j < i), computed in slices so the
    [N,C,C,K] factor tensor stays bounded."""
    N, C, K = k.shape
    Aqk = torch.zeros(N, C, C, dtype=torch.float32, device=k.device) if want_qk else None
    Mkk = torch.zeros(N, C, C, dtype=torch.float32, device=k.device)
    low = torch.tril(torch.ones(C, C, dtype=torch.bool, device=k.device))
    per = max(1, (1 << 27) // (C * C * K))
    for sl in _slices(N, per):
        d = gcv[sl, :, None, :] - gcv[sl, None, :, :]
        f = torch.exp2(torch.where(low[None, :, :, None], d, torch.full_like(d, -float("inf"))))
        if want_qk:
            Aqk[sl] = scale * torch.einsum("nik,nijk,njk->nij", q[sl], f, k[sl])
        Mkk[sl] = torch.einsum("nik,nijk,njk->nij", bk[sl], f, k[sl]) * (~torch.eye(C, dtype=torch.bool, device=k.device))
        del d, f
    return Aqk, Mkk


def _wy_scan(qf, kf, vf, gcv, bc, wc, Akk, initial_state, scale, Aqk=None, h_dtype=torch.bfloat16):
    """WY factors and the forward state scan on chunked fp32 operands
    ([B,H,NT,C,*]); also the output when Aqk is given."""
    B, H, NT, C, K = kf.shape
    V = vf.shape[-1]
    dev = kf.device
    gam = torch.exp2(gcv)
    glast = gcv[..., -1:, :]
    w_wy = Akk @ (bc * kf * gam)
    u_wy = Akk @ (wc * vf)
    qg = qf * gam
    kg = kf * torch.exp2(glast - gcv)
    lam = torch.exp2(glast[..., 0, :])                                 # [B,H,NT,K|1]
    S = torch.zeros(B, H, K, V, device=dev) if initial_state is None else initial_state.float().clone()
    hs = torch.empty(B, H, NT, K, V, device=dev, dtype=h_dtype)
    vnew = torch.empty(B, H, NT, C, V, device=dev)
    o = torch.empty(B, H, NT, C, V, device=dev) if Aqk is not None else None
    for c in range(NT):
        hb = S.to(h_dtype)
        hs[:, :, c] = hb
        Sc = hb.float()
        vn = u_wy[:, :, c] - w_wy[:, :, c] @ Sc
        vnew[:, :, c] = vn
        if o is not None:
            o[:, :, c] = scale * qg[:, :, c] @ Sc + Aqk[:, :, c] @ vn
        S = lam[:, :, c, :, None] * S + kg[:, :, c].transpose(-1, -2) @ vn
    return hs, vnew, w_wy, u_wy, qg, kg, S, o


def _family_operands(op, q, k, v, gc, beta, b, w):
    """Chunked fp32 operands: q, k, v, gate (log2 cumsum, [..,K] or [..,1]), b, w."""
    B, T, H, K = q.shape
    NT = T // CHUNK
    qf, kf, vf = (to_chunks(x.float()) for x in (q, k, v))
    if op == "delta":
        gcv = torch.zeros(B, H, NT, CHUNK, 1, device=q.device)
    elif op == "gdn":
        gcv = to_chunks(gc)[..., None]
    else:
        gcv = to_chunks(gc)
    if op == "gdn2":
        bc, wc = to_chunks(b.float()), to_chunks(w.float())
    else:
        be = to_chunks(beta.float())[..., None]
        bc, wc = be, be
    return qf, kf, vf, gcv, bc, wc


def recompute(op, q, k, v, gc, Akk, beta=None, b=None, w=None, initial_state=None):
    """Recompute w, u, qg, kg, v_new and h from saved (q, k, v, gc, Akk, gates):
    the recompute policy of FLA's chunk_<op>_bwd (recompute_w_u_fwd +
    chunk_gated_delta_rule_fwd_h, reference backends/backward.py:110-118)."""
    qf, kf, vf, gcv, bc, wc = _family_operands(op, q, k, v, gc, beta, b, w)
    A = to_chunks(Akk)
    hs, vnew, w_wy, u_wy, qg, kg, _, _ = _wy_scan(qf, kf, vf, gcv, bc, wc, A, initial_state, None)
    bf = torch.bfloat16
    return dict(w=from_chunks(w_wy).to(bf), u=from_chunks(u_wy).to(bf), qg=from_chunks(qg).to(bf),
                kg=from_chunks(kg).to(bf), v_new=from_chunks(vnew).to(bf),
                h=hs.permute(0, 2, 1, 3, 4).contiguous())


def chunk_forward(op, q, k, v, g=None, beta=None, b=None, w=None, initial_state=None,
                  scale=None, output_final_state=False, chunk=CHUNK, save=True):
    """Forward of one operator family.  Returns (o, final_state, saved dict).

    op: 'delta' | 'gdn' | 'kda' | 'gdn2'.  g is the raw per-token natural-log
    decay ([B,T,H] for gdn, [B,T,H,K] for kda/gdn2).  The saved dict holds the
    FLA-convention intermediates listed in the module docstring."""
    B, T, H, K = q.shape
    C = chunk
    assert C == CHUNK and T % C == 0, "T must be a multiple of the 64-token chunk"
    dev = q.device
    scale = K ** -0.5 if scale is None else scale
    NT = T // C
    gc = None if op == "delta" else chunk_local_cumsum(g, C)
    qf, kf, vf, gcv, bc, wc = _family_operands(op, q, k, v, gc, beta, b, w)
    bk = bc * kf
    N = B * H * NT
    if op in ("kda", "gdn2"):
        Aqk, Mkk = _pair_products(qf.reshape(N, C, K), kf.reshape(N, C, K), bk.reshape(N, C, K),
                                  gcv.reshape(N, C, K), scale)
        Aqk = Aqk.reshape(B, H, NT, C, C)
        Mkk = Mkk.reshape(B, H, NT, C, C)
    else:
        fac = torch.exp2(gcv[..., :, None, 0] - gcv[..., None, :, 0]) if op == "gdn" else 1.0
        low = torch.tril(torch.ones(C, C, dtype=torch.bool, device=dev))
        Aqk = scale * (qf @ kf.transpose(-1, -2)) * fac
        Aqk = torch.where(low, Aqk, torch.zeros((), device=dev))
        Mkk = (bk @ kf.transpose(-1, -2)) * fac
        Mkk = torch.where(torch.tril(low, -1), Mkk, torch.zeros((), device=dev))
    eye = torch.eye(C, device=dev)
    Akk = torch.linalg.solve_triangular(eye + Mkk, eye.expand_as(Mkk), upper=False, unitriangular=True)
    hs, vnew, w_wy, u_wy, qg, kg, S, o = _wy_scan(qf, kf, vf, gcv, bc, wc, Akk, initial_state, scale,
                                                  Aqk=Aqk, h_dtype=torch.bfloat16 if save else torch.float32)
    out = from_chunks(o).to(q.dtype)
    final = S if output_final_state else None
    saved = None
    if save:
        bf = torch.bfloat16
        saved = dict(
            gc=gc,
            Aqk=from_chunks(Aqk), Akk=from_chunks(Akk),
            w=from_chunks(w_wy).to(bf), u=from_chunks(u_wy).to(bf),
            qg=from_chunks(qg).to(bf), kg=from_chunks(kg).to(bf),
            v_new=from_chunks(vnew).to(bf),
            h=hs.permute(0, 2, 1, 3, 4).contiguous(),
            scale=scale,
        )
    return out, final, saved
