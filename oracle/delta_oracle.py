"""CPU float64 restatement of ReWY's chunked delta-rule backward.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``rewy_amd``) imports this
module; only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU
baseline leg may use it, and only as the checker.

Conventions (FLA's, which the reference keeps):

* tensors are T-major ``[B, T, H, D]``; per-chunk states are ``[B, NT, H, K, V]``;
* ``g`` handed to the public operators is the per-token *natural-log* decay;
  the backward kernels receive the chunk-local cumsum in *log2* units
  (``chunk_local_cumsum(g, scale=RCP_LN2)``, reference ``_compat/gdn.py:63-69``);
* one generic family description covers all four operators::

      delta : g = 0,             b = beta (broadcast K), w = beta (broadcast V)
      gdn   : g scalar per token, b = beta,               w = beta
      kda   : g vector [K],       b = beta,               w = beta
      gdn2  : g vector [K],       b [K] erase gate,       w [V] write gate

  with the token recurrence (reference ``validation.py:23-38``,
  ``benchmarks/plotting/check_manuscript_math.py:11-19``)::

      S <- diag(exp(g_t)) S
      r  = w_t * v_t - S^T (b_t * k_t)
      S <- S + k_t r^T
      o_t = scale * S^T q_t

Functions and what pins them (see ``tests/test_oracle.py``):

* ``recurrence``              -- textbook statement; pinned by torch fp64 autograd
                                 and by the chunked forward.
* ``torch_token_recurrence``  -- the reference's CPU path (``validation.py:23-38``) in
                                 torch, batched; pinned by equality of its fp64
                                 autograd with ``backward``.
* ``chunk_pullback``          -- closed-form single-chunk backward, restating
                                 ``check_manuscript_math.py:21-54``; pinned by
                                 complex-step differentiation of ``recurrence``.
* ``forward`` / ``backward``  -- vectorised multi-chunk chain
                                 (``check_manuscript_math.py:102-124``); pinned by
                                 complex step and by ``chunk_pullback`` chaining.
* ``stage_*``                 -- the same backward split at the HIP kernel
                                 boundaries (state recurrence, residual-WY +
                                 matrix intra), in FLA's log2 / pairwise form;
                                 pinned by equality with ``backward``.
* ``intra_pairwise``          -- explicit pairwise matrix-intra oracle restating
                                 ``scripts/npu950_intra_regression.py:25-46``;
                                 pinned by central finite differences of the
                                 scalar objective (``tests/test_npu950.py:52-98``)
                                 and by the centred-factor identity
                                 (``check_operator_identities.py:31-43``).
"""
from __future__ import annotations

import numpy as np

LN2 = float(np.log(2.0))
FAMILIES = ("delta", "gdn", "kda", "gdn2")


# --------------------------------------------------------------------------
# token recurrence (one sequence-head), dtype-generic so complex step works
# --------------------------------------------------------------------------
def recurrence(q, k, v, g, b, w, S0, scale=1.0):
    """o [T,V], final state [K,V] of the delta rule; g natural-log [T,K]."""
    S = S0.copy()
    out = []
    for t in range(q.shape[0]):
        S = np.exp(g[t])[:, None] * S
        r = w[t] * v[t] - S.T @ (b[t] * k[t])
        S = S + np.outer(k[t], r)
        out.append(scale * (S.T @ q[t]))
    return np.asarray(out), S


def torch_token_recurrence(op, xs):
    """The reference's CPU path (validation.py:23-38): the token recurrence of ``op`` over a
    batch in torch (any dtype; fp64 there), differentiable by autograd.  ``xs``: q, k, v
    [B,T,H,K], initial_state [B,H,K,V], g (natural log; [B,T,H] for gdn, [B,T,H,K] for kda /
    gdn2, absent for delta), beta [B,T,H] or (gdn2) b [B,T,H,K], w [B,T,H,V].  Returns (o, S_T).
    Pinned against ``backward`` (complex-step pinned) by tests/test_oracle.py."""
    import torch
    q, k, v = xs["q"], xs["k"], xs["v"]
    S = xs["initial_state"]
    ys = []
    for i in range(k.shape[1]):
        if op != "delta":
            gi = xs["g"][:, i]
            if op == "gdn":
                gi = gi[..., None]
            S = S * gi.exp()[..., None]
        kt = k[:, i]
        if op == "gdn2":
            r = xs["w"][:, i] * v[:, i] - torch.einsum("bhk,bhkv->bhv", xs["b"][:, i] * kt, S)
        else:
            r = xs["beta"][:, i, ..., None] * (v[:, i] - torch.einsum("bhk,bhkv->bhv", kt, S))
        S = S + kt[..., None] * r[..., None, :]
        ys.append(torch.einsum("bhk,bhkv->bhv", q[:, i] * q.shape[-1] ** -.5, S))
    return torch.stack(ys, 1), S


def recurrence_objective(q, k, v, g, b, w, S0, dO, dS, scale=1.0):
    o, S = recurrence(q, k, v, g, b, w, S0, scale)
    return np.sum(o * dO) + np.sum(S * dS)


# --------------------------------------------------------------------------
# closed-form single-chunk backward (check_manuscript_math.py:21-54)
# --------------------------------------------------------------------------
def chunk_pullback(Q, K, V, g, b, w, S, dO, dS):
    """Gradients of <o,dO> + <S_end,dS> for one chunk whose queries already carry
    the score scale.  Returns ([dQ,dK,dV,dg,db,dw,dS_in], aux) with g natural-log
    per token (the reverse cumsum is applied here)."""
    n = Q.shape[0]
    G = np.cumsum(g, axis=0)
    gam = np.exp(G)
    lam = gam[-1]
    E = b * K * gam           # erase direction, gate-weighted
    Y = K / gam               # key, inverse-gate weighted
    Z = w * V                 # written value
    Qg = Q * gam
    A = np.linalg.inv(np.eye(n) + np.tril(E @ Y.T, -1))
    R = A @ (Z - E @ S)                       # v_new
    C = np.tril(Qg @ Y.T)                     # intra-chunk scores (Aqk)
    dR = C.T @ dO + (Y * lam) @ dS             # residual adjoint
    Hm = np.tril(dO @ R.T)                    # adjoint of C
    P = A.T @ dR                              # residual product 1
    D = -np.tril(P @ R.T, -1)                 # residual product 2
    dQg = dO @ S.T + Hm @ Y
    dE = -P @ S.T + D @ Y                     # residual product 3 enters here
    fb = R @ dS.T
    dY = Hm.T @ Qg + D.T @ E + fb * lam
    dS_in = Qg.T @ dO + lam[:, None] * dS - E.T @ P
    dQ = gam * dQg
    dK = gam * b * dE + dY / gam
    db = gam * K * dE
    dV = w * P
    dw = V * P
    dG = Qg * dQg + E * dE - Y * dY
    dG[-1] += lam * ((S * dS).sum(1) + (Y * fb).sum(0))
    dg = np.cumsum(dG[::-1], axis=0)[::-1]
    return [dQ, dK, dV, dg, db, dw, dS_in], dict(P=P, R=R, D=D, A=A, H=Hm)


def partitioned_pullback(q, k, v, g, b, w, S0, dO, dS, lengths, scale=1.0):
    """Chain chunk pullbacks through the boundary states obtained from the token
    recurrence (check_manuscript_math.py:102-124).  Returns
    [dq, dk, dv, dg, db, dw, dS0]."""
    starts = np.cumsum([0] + list(lengths))
    state = S0.copy()
    incoming = []
    for lo, hi in zip(starts[:-1], starts[1:]):
        incoming.append(state.copy())
        _, state = recurrence(q[lo:hi], k[lo:hi], v[lo:hi], g[lo:hi], b[lo:hi], w[lo:hi], state)
    grads = [np.zeros_like(x) for x in (q, k, v, g, b, w)]
    terminal = dS.copy()
    for c in reversed(range(len(lengths))):
        lo, hi = starts[c], starts[c + 1]
        got, _ = chunk_pullback(q[lo:hi] * scale, k[lo:hi], v[lo:hi], g[lo:hi], b[lo:hi],
                                w[lo:hi], incoming[c], dO[lo:hi], terminal)
        got[0] = got[0] * scale
        for a in range(6):
            grads[a][lo:hi] = got[a]
        terminal = got[6]
    return grads + [terminal]


# --------------------------------------------------------------------------
# family plumbing on [B,T,H,D] arrays
# --------------------------------------------------------------------------
def family_gates(op, q, v, g=None, beta=None, b=None, w=None):
    """Map operator inputs to the generic (g [B,T,H,K], b [B,T,H,K], w [B,T,H,V])."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    if op == "delta":
        gv = np.zeros((B, T, H, K))
    elif op == "gdn":
        gv = np.broadcast_to(np.asarray(g, np.float64)[..., None], (B, T, H, K)).copy()
    else:
        gv = np.asarray(g, np.float64)
    if op == "gdn2":
        bv, wv = np.asarray(b, np.float64), np.asarray(w, np.float64)
    else:
        be = np.asarray(beta, np.float64)[..., None]
        bv = np.broadcast_to(be, (B, T, H, K)).copy()
        wv = np.broadcast_to(be, (B, T, H, V)).copy()
    return gv, bv, wv


def _to_chunks(x, C):
    """[B,T,H,D] -> [B,H,NT,C,D]"""
    B, T, H = x.shape[:3]
    return np.ascontiguousarray(x.reshape(B, T // C, C, H, *x.shape[3:]).transpose(0, 3, 1, 2, *range(4, x.ndim + 1)))


def _from_chunks(x):
    """[B,H,NT,C,D] -> [B,T,H,D]"""
    B, H, NT, C = x.shape[:4]
    return np.ascontiguousarray(x.transpose(0, 2, 3, 1, *range(4, x.ndim)).reshape(B, NT * C, H, *x.shape[4:]))


def _tril(x, k=0):
    n = x.shape[-1]
    return x * np.tri(n, n, k, dtype=bool)


def _T(x):
    return np.swapaxes(x, -1, -2)


def forward(op, q, k, v, g=None, beta=None, b=None, w=None, h0=None, scale=None, chunk=64):
    """Vectorised fp64 chunk forward for all families.  Returns a dict holding o,
    the final state and FLA-convention intermediates (gc in log2 units, Aqk with
    the scale folded in, Akk, w/u of the WY form, qg, kg, v_new, per-chunk
    states h [B,NT,H,K,V])."""
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    B, T, H, K = q.shape
    V = v.shape[-1]
    assert T % chunk == 0
    scale = K ** -0.5 if scale is None else scale
    gv, bv, wv = family_gates(op, q, v, g, beta, b, w)
    Q, Kc, Vc, Gr, Bc, Wc = (_to_chunks(x, chunk) for x in (q, k, v, gv, bv, wv))
    G = np.cumsum(Gr, axis=3)
    gam = np.exp(G)
    lam = gam[..., -1, :]                               # [B,H,NT,K]
    # pairwise gate factors keep everything finite in fp64 for any chunk span
    fac = np.exp(np.where(np.tri(chunk, dtype=bool)[..., None],
                          G[..., :, None, :] - G[..., None, :, :], -np.inf))  # [B,H,NT,C,C,K]
    Akk = np.linalg.inv(np.eye(chunk) + np.einsum("...ik,...jk,...ijk->...ij", Bc * Kc, Kc,
                                                  fac * ~np.eye(chunk, dtype=bool)[..., None]))
    Aqk = scale * np.einsum("...ik,...jk,...ijk->...ij", Q, Kc, fac)
    Wwy = Akk @ (Bc * Kc * gam)
    Uwy = Akk @ (Wc * Vc)
    kg = Kc * np.exp(G[..., -1:, :] - G)
    S = np.zeros((B, H, K, V)) if h0 is None else np.asarray(h0, np.float64).copy()
    NT = T // chunk
    hs = np.zeros((B, H, NT, K, V))
    R = np.zeros_like(Vc)
    for c in range(NT):
        hs[:, :, c] = S
        R[:, :, c] = Uwy[:, :, c] - Wwy[:, :, c] @ S
        S = lam[:, :, c, :, None] * S + _T(kg[:, :, c]) @ R[:, :, c]
    o = scale * (Q * gam) @ hs + Aqk @ R
    return dict(o=_from_chunks(o), final=S, gc=_from_chunks(G / LN2), G=G,
                Aqk=_from_chunks(Aqk), Akk=_from_chunks(Akk), w=_from_chunks(Wwy),
                u=_from_chunks(Uwy), qg=_from_chunks(Q * gam), kg=_from_chunks(kg),
                v_new=_from_chunks(R), h=np.ascontiguousarray(hs.transpose(0, 2, 1, 3, 4)),
                scale=scale, chunk=chunk)


def backward(op, q, k, v, g=None, beta=None, b=None, w=None, h0=None, dO=None, dht=None,
             scale=None, chunk=64):
    """End-to-end fp64 gradients of <o,dO> + <S_T,dht> with respect to the public
    operator inputs.  Returns a dict with dq, dk, dv, dg (raw natural-log gate,
    scalar for gdn, absent for delta), dbeta (scalar-beta families) or db/dw
    (gdn2), dh0.  Vectorised over chunks; the chunk formulas are
    ``chunk_pullback``'s, with every exp(G_i - G_j) formed pairwise so the
    result stays finite for any gate span."""
    fw = forward(op, q, k, v, g, beta, b, w, h0, scale, chunk)
    scale = fw["scale"]
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // chunk
    gv, bv, wv = family_gates(op, q, v, g, beta, b, w)
    Q, Kc, Vc, Bc, Wc, dOc = (_to_chunks(x, chunk) for x in (q, k, v, bv, wv, np.asarray(dO, np.float64)))
    G = fw["G"]
    gam = np.exp(G)
    lam = gam[..., -1, :]
    A = _to_chunks(fw["Akk"], chunk)
    Aqk = _to_chunks(fw["Aqk"], chunk)
    R = _to_chunks(fw["v_new"], chunk)
    Wwy = _to_chunks(fw["w"], chunk)
    kg = _to_chunks(fw["kg"], chunk)
    hs = fw["h"].transpose(0, 2, 1, 3, 4)               # [B,H,NT,K,V]
    # reverse state recurrence
    dv_local = _T(Aqk) @ dOc
    dh = np.zeros((B, H, NT, K, V))
    dR = np.zeros_like(R)
    state = np.zeros((B, H, K, V)) if dht is None else np.asarray(dht, np.float64).copy()
    for c in reversed(range(NT)):
        dh[:, :, c] = state
        dR[:, :, c] = kg[:, :, c] @ state + dv_local[:, :, c]
        state = (lam[:, :, c, :, None] * state + scale * _T(Q[:, :, c] * gam[:, :, c]) @ dOc[:, :, c]
                 - _T(Wwy[:, :, c]) @ dR[:, :, c])
    dh0 = state
    post = _post(Q, Kc, Vc, G, Bc, Wc, A, hs, dh, R, dOc, dR, scale, chunk)
    dG = post["dG"]
    dgraw = np.cumsum(dG[..., ::-1, :], axis=3)[..., ::-1, :]
    out = dict(dq=_from_chunks(post["dq"]), dk=_from_chunks(post["dk"]),
               dv=_from_chunks(post["dv"]), dh0=dh0)
    db, dw = _from_chunks(post["db"]), _from_chunks(post["dw"])
    if op == "gdn2":
        out["db"], out["dw"] = db, dw
    else:
        out["dbeta"] = db.sum(-1) + dw.sum(-1)
    if op in ("kda", "gdn2"):
        out["dg"] = _from_chunks(dgraw)
    elif op == "gdn":
        out["dg"] = _from_chunks(dgraw).sum(-1)
    out["fwd"] = fw
    out["stage"] = dict(dh=np.ascontiguousarray(dh.transpose(0, 2, 1, 3, 4)),
                        dR=_from_chunks(dR), dv_local=_from_chunks(dv_local),
                        P=_from_chunks(post["P"]), D=_from_chunks(post["D"]),
                        dAqk=_from_chunks(post["L"]), dG=_from_chunks(dG))
    return out


def _post(Q, Kc, Vc, G, Bc, Wc, A, hs, dh, R, dOc, dR, scale, chunk):
    """Chunk-parallel part of the backward (residual WY + matrix intra + state
    gradient epilogue) in pairwise-gated form.  Q is unscaled."""
    gam = np.exp(G)
    lam = gam[..., -1, :]
    low = np.tri(chunk, dtype=bool)
    fac = np.exp(np.where(low[..., None], G[..., :, None, :] - G[..., None, :, :], -np.inf))
    L = scale * _tril(dOc @ _T(R))                      # dAqk
    P = _T(A) @ dR                                      # residual product 1
    D = -_tril(P @ _T(R), -1)                           # residual product 2
    Ebar = -(P @ _T(hs))                                # residual product 3 (E-bar direct)
    dq_s = (dOc @ _T(hs)) * gam * scale
    dk_s = (R @ _T(dh)) * np.exp(G[..., -1:, :] - G)
    uq = np.einsum("...ij,...jk,...ijk->...ik", L, Kc, fac)
    ue = np.einsum("...ij,...jk,...ijk->...ik", D, Kc, fac)
    uk = (np.einsum("...ji,...jk,...jik->...ik", L, Q, fac)
          + np.einsum("...ji,...jk,...jik->...ik", D, Bc * Kc, fac))
    dq = dq_s + uq
    dk = dk_s + Bc * gam * Ebar + Bc * ue + uk
    dv = Wc * P
    dw = Vc * P
    db = Kc * gam * Ebar + Kc * ue
    dG = Q * dq - Kc * dk_s + Bc * Kc * gam * Ebar + Kc * (Bc * ue - uk)
    dG[..., -1, :] += lam * (hs * dh).sum(-1) + (Kc * dk_s).sum(-2)
    return dict(dq=dq, dk=dk, dv=dv, dw=dw, db=db, dG=dG, P=P, D=D, L=L)


# --------------------------------------------------------------------------
# stage oracles at the HIP kernel boundaries (FLA conventions, log2 gates)
# --------------------------------------------------------------------------
def stage_state_bwd(qg, kg, w, gc, dO, dv_local, dht=None, h0_present=True, scale=1.0, chunk=64):
    """Reverse inter-chunk state recurrence (reference vector_state_gpu.py:28-43,
    FLA chunk_gated_delta_rule_bwd_dhu).  qg/kg carry the gate weighting; gc is
    the log2 chunk-local cumsum [B,T,H,K].  Returns dh [B,NT,H,K,V], dR, dh0."""
    qg, kg, w, gc, dO, dv_local = (np.asarray(x, np.float64) for x in (qg, kg, w, gc, dO, dv_local))
    B, T, H, K = qg.shape
    V = dO.shape[-1]
    NT = T // chunk
    Qc, Kc, Wc, Gc, dOc, dvc = (_to_chunks(x, chunk) for x in (qg, kg, w, gc, dO, dv_local))
    lam = np.exp2(Gc[..., -1, :])
    state = np.zeros((B, H, K, V)) if dht is None else np.asarray(dht, np.float64).copy()
    dh = np.zeros((B, H, NT, K, V))
    dR = np.zeros_like(dvc)
    for c in reversed(range(NT)):
        dh[:, :, c] = state
        dR[:, :, c] = Kc[:, :, c] @ state + dvc[:, :, c]
        state = lam[:, :, c, :, None] * state + scale * _T(Qc[:, :, c]) @ dOc[:, :, c] - _T(Wc[:, :, c]) @ dR[:, :, c]
    return np.ascontiguousarray(dh.transpose(0, 2, 1, 3, 4)), _from_chunks(dR), state


def stage_post(op, q, k, v, gc, beta=None, b=None, w=None, Akk=None, h=None, dh=None,
               v_new=None, dO=None, dR=None, scale=1.0, chunk=64):
    """Fused residual-WY + matrix-intra + epilogue stage (reference
    kda_residual_tri_beta.py:8-73, kda_residual_local_beta_consumer.py:23-180,
    endpoint_intra.py:16-297, gdn2_consumer_fp32.py:8-75,
    scalar_liveness_gpu.py:12-84).  gc is the log2 chunk-local cumsum (scalar
    [B,T,H] for gdn, absent for delta).  Returns dq, dk, dv, dg (after the
    in-chunk reverse cumsum, still in the log2-cumsum parameterisation's
    natural-log gradient, i.e. the gradient of the raw per-token gate), and
    dbeta or db/dw."""
    q, k, v, dO, dR, v_new = (np.asarray(x, np.float64) for x in (q, k, v, dO, dR, v_new))
    B, T, H, K = q.shape
    if op == "delta":
        G = np.zeros((B, T, H, K))
    else:
        gc = np.asarray(gc, np.float64) * LN2
        G = np.broadcast_to(gc[..., None], (B, T, H, K)).copy() if op == "gdn" else gc
    _, bv, wv = family_gates(op, q, v, None, beta, b, w)
    Q, Kc, Vc, Gc, Bc, Wc, Ac, dOc, dRc, Rc = (
        _to_chunks(x, chunk) for x in (q, k, v, G, bv, wv, np.asarray(Akk, np.float64), dO, dR, v_new))
    hs = np.asarray(h, np.float64).transpose(0, 2, 1, 3, 4)
    dhs = np.asarray(dh, np.float64).transpose(0, 2, 1, 3, 4)
    post = _post(Q, Kc, Vc, Gc, Bc, Wc, Ac, hs, dhs, Rc, dOc, dRc, scale, chunk)
    dG = post["dG"]
    dgraw = _from_chunks(np.cumsum(dG[..., ::-1, :], axis=3)[..., ::-1, :])
    out = dict(dq=_from_chunks(post["dq"]), dk=_from_chunks(post["dk"]), dv=_from_chunks(post["dv"]))
    db, dw = _from_chunks(post["db"]), _from_chunks(post["dw"])
    if op == "gdn2":
        out["db"], out["dw"] = db, dw
    else:
        out["dbeta"] = db.sum(-1) + dw.sum(-1)
    if op in ("kda", "gdn2"):
        out["dg"] = dgraw
    elif op == "gdn":
        out["dg"] = dgraw.sum(-1)
    return out


# --------------------------------------------------------------------------
# explicit pairwise matrix-intra oracle (scripts/npu950_intra_regression.py:25-46)
# --------------------------------------------------------------------------
def intra_pairwise(q, k, g, beta, dAqk, dAkk, dq, dk, db, dg, vector_beta=False):
    """Adds the matrix-intra VJP into (dq, dk, db, dg) for inputs [B,T,H,*] with
    g in log2 units (one chunk = the whole T axis).  dAqk is used lower-inclusive,
    dAkk strictly lower.  Returns new arrays; inputs are not modified."""
    q, k, g, beta, L, Dm = (np.asarray(x, np.float64) for x in (q, k, g, beta, dAqk, dAkk))
    outs = [np.asarray(x, np.float64).copy() for x in (dq, dk, db, dg)]
    B, T, H, K = q.shape
    low = np.tri(T, dtype=bool)
    for bb in range(B):
        for hh in range(H):
            gh = g[bb, :, hh]
            fac = np.exp2(np.where(low[:, :, None], gh[:, None, :] - gh[None, :, :], -np.inf))
            l = np.tril(L[bb, :, hh])
            d = np.tril(Dm[bb, :, hh], -1)
            be = beta[bb, :, hh] if vector_beta else beta[bb, :, hh, None]
            kk, qq = k[bb, :, hh], q[bb, :, hh]
            uq = np.einsum("ij,ijk,jk->ik", l, fac, kk)
            ue = np.einsum("ij,ijk,jk->ik", d, fac, kk)
            uk = np.einsum("ji,jik,jk->ik", l, fac, qq) + np.einsum("ji,jik,jk->ik", d, fac, kk * be)
            outs[0][bb, :, hh] += uq
            outs[1][bb, :, hh] += be * ue + uk
            outs[2][bb, :, hh] += ue * kk if vector_beta else (ue * kk).sum(-1)
            outs[3][bb, :, hh] += qq * uq + kk * (be * ue - uk)
    return outs


def intra_objective(q, k, gate, beta, l, d):
    """Independent scalar forward whose gradient the intra VJP is (natural-log
    gate; restates tests/test_npu950.py:52-62)."""
    value = 0.0
    for i in range(len(q)):
        for j in range(i + 1):
            f = np.exp(gate[i] - gate[j])
            value += l[i, j] * np.sum(q[i] * k[j] * f)
            if j < i:
                value += d[i, j] * np.sum(beta[i] * k[i] * k[j] * f)
    return value


# --------------------------------------------------------------------------
# error metric (reference validation.py:40-45, run_cuda.py:53-60)
# --------------------------------------------------------------------------
def error(ref, got, limit):
    ref = np.asarray(ref, np.float64)
    got = np.asarray(got, np.float64)
    diff = got - ref
    absolute = float(np.abs(diff).max()) if diff.size else 0.0
    relative = float(np.linalg.norm(diff) / max(np.linalg.norm(ref), 1e-30))
    finite = bool(np.isfinite(got).all())
    small = float(np.abs(ref).max()) < 1e-6 if ref.size else True
    passed = finite and (absolute <= 1e-6 if small else relative <= limit)
    return dict(relative_l2=relative, max_abs=absolute, limit=limit, passed=passed)


def limit_for(name):
    """rel-L2 budget per gradient (reference validation.py:68)."""
    return 0.02 if name in ("dg", "dbeta", "db", "dw", "g", "beta", "b", "w") else 0.008


def dv_local(Aqk, dO, chunk=64):
    """Aqk^T dO per chunk (FLA chunk_kda_bwd_dAv / chunk_bwd_dv_local output)."""
    A = _to_chunks(np.asarray(Aqk, np.float64), chunk)
    d = _to_chunks(np.asarray(dO, np.float64), chunk)
    return _from_chunks(_T(A) @ d)
