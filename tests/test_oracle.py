"""Pins of the fp64 oracle (CPU only).

Each check is independent of the formula it tests: complex-step derivatives
of the token recurrence (reference benchmarks/plotting/check_manuscript_math.py:56-101),
torch fp64 autograd of the recurrence (reference validation.py:23-38),
partition invariance (check_manuscript_math.py:102-169), central finite
differences of the intra objective (tests/test_npu950.py:52-98), the
centred-factor and Gram identities (check_operator_identities.py,
check_manuscript_math.py:171-179) and the reference's real captured intra
inputs (validation/npu950_intra, copied under tests/golden).
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import delta_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def _family_inputs(rng, family, n, K, V):
    Q = rng.normal(size=(n, K)) * .3
    Kk = rng.normal(size=(n, K)) * .2
    Vv = rng.normal(size=(n, V))
    S = rng.normal(size=(K, V)) * .2
    g = rng.uniform(-.3, .08, size=(n, K))
    if family == "delta":
        g[:] = 0
    if family == "gdn":
        g[:] = g[:, :1]
    beta = rng.uniform(.1, .9, size=(n, 1))
    beta[0] = 0
    b = np.broadcast_to(beta, (n, K)).copy()
    w = np.broadcast_to(beta, (n, V)).copy()
    if family == "gdn2":
        b = rng.uniform(-.1, .9, size=(n, K))
        w = rng.uniform(-.1, .9, size=(n, V))
    return [Q, Kk, Vv, g, b, w, S]


def _complex_step(inputs, dO, dS, idx_arg, idx):
    pert = [z.astype(complex) for z in inputs]
    pert[idx_arg][idx] += 1e-25j
    return O.recurrence_objective(*pert, dO, dS).imag / 1e-25


@pytest.mark.parametrize("family", O.FAMILIES)
@pytest.mark.parametrize("n,K,V", [(1, 3, 2), (4, 3, 5), (7, 5, 3)])
def test_chunk_pullback_matches_complex_step(family, n, K, V):
    rng = np.random.default_rng(79 + n)
    inputs = _family_inputs(rng, family, n, K, V)
    dO = rng.normal(size=(n, V))
    dS = rng.normal(size=(K, V))
    got, aux = O.chunk_pullback(*inputs, dO, dS)
    err = 0.0
    for a, x in enumerate(inputs):
        for idx in np.ndindex(x.shape):
            err = max(err, abs(_complex_step(inputs, dO, dS, a, idx) - got[a][idx]))
    assert err < 1e-11, err
    if family != "gdn2":
        # residual identity: beta * dbeta = sum_v P * R (kda_residual_tri_beta.py:50-60)
        beta = inputs[4][:, 0]
        dbeta = got[4].sum(1) + got[5].sum(1)
        assert np.max(np.abs(beta * dbeta - (aux["P"] * aux["R"]).sum(1))) < 1e-11


@pytest.mark.parametrize("family", O.FAMILIES)
def test_vectorised_backward_matches_partitioned_pullback_and_complex_step(family):
    rng = np.random.default_rng(5)
    B, T, H, K, V, C = 1, 8, 2, 3, 4, 4
    q = rng.normal(size=(B, T, H, K))
    k = rng.normal(size=(B, T, H, K)) * .5
    v = rng.normal(size=(B, T, H, V))
    g = rng.uniform(-.5, 0, (B, T, H, K)) if family in ("kda", "gdn2") else rng.uniform(-.5, 0, (B, T, H))
    beta = rng.uniform(.1, .9, (B, T, H))
    beta[:, ::3] = 0
    b = rng.uniform(.1, .9, (B, T, H, K))
    w = rng.uniform(.1, .9, (B, T, H, V))
    h0 = rng.normal(size=(B, H, K, V)) * .2
    dO = rng.normal(size=(B, T, H, V))
    dht = rng.normal(size=(B, H, K, V))
    out = O.backward(family, q, k, v, g=g, beta=beta, b=b, w=w, h0=h0, dO=dO, dht=dht, scale=.7, chunk=C)
    gv, bv, wv = O.family_gates(family, q, v, g, beta, b, w)
    for hh in range(H):
        args = [x[0, :, hh] for x in (q, k, v, gv, bv, wv)]
        ref = O.partitioned_pullback(*args, h0[0, hh], dO[0, :, hh], dht[0, hh], [C] * (T // C), scale=.7)
        np.testing.assert_allclose(out["dq"][0, :, hh], ref[0], atol=1e-12)
        np.testing.assert_allclose(out["dk"][0, :, hh], ref[1], atol=1e-12)
        np.testing.assert_allclose(out["dv"][0, :, hh], ref[2], atol=1e-12)
        np.testing.assert_allclose(out["dh0"][0, hh], ref[6], atol=1e-12)
        if family in ("kda", "gdn2"):
            np.testing.assert_allclose(out["dg"][0, :, hh], ref[3], atol=1e-12)
        if family == "gdn":
            np.testing.assert_allclose(out["dg"][0, :, hh], ref[3].sum(-1), atol=1e-12)
        if family == "gdn2":
            np.testing.assert_allclose(out["db"][0, :, hh], ref[4], atol=1e-12)
            np.testing.assert_allclose(out["dw"][0, :, hh], ref[5], atol=1e-12)
        else:
            np.testing.assert_allclose(out["dbeta"][0, :, hh], ref[4].sum(-1) + ref[5].sum(-1), atol=1e-12)
        o, S = O.recurrence(*args, h0[0, hh], .7)
        np.testing.assert_allclose(out["fwd"]["o"][0, :, hh], o, atol=1e-12)
        np.testing.assert_allclose(out["fwd"]["final"][0, hh], S, atol=1e-12)
    # complex step straight on the public-input gradients of one head, q and g
    hh = 0
    args = [x[0, :, hh] for x in (q, k, v, gv, bv, wv)] + [h0[0, hh]]
    scaled = list(args)
    scaled[0] = args[0] * .7
    for idx in [(0, 0), (5, 2), (7, 1)]:
        d = _complex_step(scaled, dO[0, :, hh], dht[0, hh], 0, idx) * .7
        assert abs(d - out["dq"][0, idx[0], hh, idx[1]]) < 1e-11
        if family in ("kda", "gdn2"):
            d = _complex_step(scaled, dO[0, :, hh], dht[0, hh], 3, idx)
            assert abs(d - out["dg"][0, idx[0], hh, idx[1]]) < 1e-11


@pytest.mark.parametrize("family", O.FAMILIES)
def test_backward_matches_torch_autograd_of_token_recurrence(family):
    """Independent check at the real head size (K = V = 128) over two chunks."""
    import torch
    from tests._inputs import make_inputs
    xs, dO = make_inputs(family, 1, 128, 2, seed=4)
    n = lambda x: None if x is None else x.double().numpy()
    out = O.backward(family, n(xs["q"]), n(xs["k"]), n(xs["v"]), g=n(xs.get("g")), beta=n(xs.get("beta")),
                     b=n(xs.get("b")), w=n(xs.get("w")), h0=n(xs["initial_state"]), dO=n(dO), dht=None)
    t = {k: v.double().clone().requires_grad_() for k, v in xs.items()}
    o, _ = O.torch_token_recurrence(family, t)
    grads = torch.autograd.grad(o, tuple(t.values()), dO.double())
    names = {"q": "dq", "k": "dk", "v": "dv", "g": "dg", "beta": "dbeta", "b": "db", "w": "dw",
             "initial_state": "dh0"}
    for (name, _), gr in zip(t.items(), grads):
        np.testing.assert_allclose(out[names[name]], gr.numpy(), rtol=1e-9, atol=1e-10, err_msg=name)


@pytest.mark.parametrize("family", O.FAMILIES)
def test_stage_functions_compose_to_backward(family):
    from tests._inputs import make_inputs
    xs, dO = make_inputs(family, 1, 128, 2, seed=9, beta_zero_every=5 if family != "gdn2" else 0)
    n = lambda x: None if x is None else x.double().numpy()
    dht = np.random.default_rng(2).normal(size=(1, 2, 128, 128)) * .1
    out = O.backward(family, n(xs["q"]), n(xs["k"]), n(xs["v"]), g=n(xs.get("g")), beta=n(xs.get("beta")),
                     b=n(xs.get("b")), w=n(xs.get("w")), h0=n(xs["initial_state"]), dO=n(dO), dht=dht)
    fw = out["fwd"]
    gcv = fw["gc"]
    if family == "delta":
        gcs = None
    elif family == "gdn":
        gcs = gcv[..., 0]
    else:
        gcs = gcv
    dvl = O.dv_local(fw["Aqk"], n(dO))
    dh, dR, dh0 = O.stage_state_bwd(fw["qg"], fw["kg"], fw["w"], gcv, n(dO), dvl, dht=dht, scale=fw["scale"])
    np.testing.assert_allclose(dh0, out["dh0"], atol=1e-10)
    post = O.stage_post(family, n(xs["q"]), n(xs["k"]), n(xs["v"]), gcs, beta=n(xs.get("beta")), b=n(xs.get("b")),
                        w=n(xs.get("w")), Akk=fw["Akk"], h=fw["h"], dh=dh, v_new=fw["v_new"], dO=n(dO), dR=dR,
                        scale=fw["scale"])
    for name in ("dq", "dk", "dv", "dg", "dbeta", "db", "dw"):
        if name in out:
            np.testing.assert_allclose(post[name], out[name], atol=1e-10, err_msg=name)


def test_residual_triple_equals_seven_product_formulation():
    """D = -L<(P R^T) with P = A^T dR equals -L<(J A^T), J = A^T (dR Z^T + Wb E^T),
    Wb = -dR S^T: the 3-product and 7-product DAGs of intro_graph_data.json."""
    rng = np.random.default_rng(0)
    for n, K, V in [(4, 3, 5), (16, 8, 8), (64, 16, 16)]:
        E = rng.normal(size=(n, K)) * .3
        Y = rng.normal(size=(n, K)) * .3
        Z = rng.normal(size=(n, V))
        S = rng.normal(size=(K, V))
        dR = rng.normal(size=(n, V))
        A = np.linalg.inv(np.eye(n) + np.tril(E @ Y.T, -1))
        R = A @ (Z - E @ S)
        P = A.T @ dR
        D3 = -np.tril(P @ R.T, -1)
        Wb = -dR @ S.T
        J = A.T @ (dR @ Z.T + Wb @ E.T)
        D7 = -np.tril(J @ A.T, -1)
        np.testing.assert_allclose(D3, D7, atol=1e-10)
        np.testing.assert_allclose(A.T @ Wb, -P @ S.T, atol=1e-10)   # E-bar direct


def test_gram_elimination_identity():
    """check_manuscript_math.py:171-179: the Gram-free gate gradient."""
    rng = np.random.default_rng(1)
    for n, k in [(1, 2), (4, 3), (7, 5), (64, 128)]:
        K = rng.normal(size=(n, k))
        G = rng.normal(size=(n, n))
        beta = rng.normal(size=n)
        beta[0] = 0
        J = beta[:, None] * G * (K @ K.T)
        L = G @ K
        R = G.T @ (beta[:, None] * K)
        new = beta * (K * L).sum(1) - (K * R).sum(1)
        np.testing.assert_allclose(new, J.sum(1) - J.sum(0), atol=1e-9)


@pytest.mark.parametrize("vector_beta", [False, True])
@pytest.mark.parametrize("span", [3., 96.])
def test_intra_oracle_against_finite_differences(vector_beta, span):
    """Restates tests/test_npu950.py:52-98 for intra_pairwise (gates in log2 units)."""
    rng = np.random.default_rng(950)
    c, kdim = 16, 32
    q, k = rng.normal(size=(2, c, kdim))
    gate = -np.linspace(0., span * np.log(2), c)[:, None] * np.ones((1, kdim))
    beta = rng.uniform(.1, .9, (c, kdim if vector_beta else 1))
    beta[::3] = 0.
    l = np.tril(rng.normal(size=(c, c)))
    d = np.tril(rng.normal(size=(c, c)), -1)
    z = lambda *s: np.zeros(s)
    be = beta if vector_beta else beta[:, 0]
    outs = O.intra_pairwise(q[None, :, None], k[None, :, None], (gate / np.log(2))[None, :, None],
                            be[None, :, None], l[None, :, None], d[None, :, None],
                            z(1, c, 1, kdim), z(1, c, 1, kdim), z(1, c, 1, kdim) if vector_beta else z(1, c, 1),
                            z(1, c, 1, kdim), vector_beta=vector_beta)
    dq, dk, db, dg = (x[0, :, 0] for x in outs)
    gradients = (dq, dk, dg, db if vector_beta else db[:, None])
    inputs = (q, k, gate, beta)
    for i, grad in enumerate(gradients):
        direction = rng.normal(size=inputs[i].shape)
        pos, neg = list(inputs), list(inputs)
        eps = 1e-5
        pos[i] = inputs[i] + eps * direction
        neg[i] = inputs[i] - eps * direction
        numerical = (O.intra_objective(*pos, l, d) - O.intra_objective(*neg, l, d)) / (2 * eps)
        np.testing.assert_allclose(numerical, np.sum(grad * direction), rtol=2e-6, atol=2e-6)


def test_centred_and_block_anchored_factors_are_invariant():
    """check_operator_identities.py:31-43: rescaling by any per-column anchor leaves
    the intra outputs unchanged (the identity the kernels' anchors rely on)."""
    rng = np.random.default_rng(20261025)
    n, d = 16, 8
    G = -np.cumsum(rng.uniform(0, 2, (n, d)), 0)
    Q, K, Be = rng.normal(size=(3, n, d))
    Hm, Dm = np.tril(rng.normal(size=(n, n))), np.tril(rng.normal(size=(n, n)), -1)
    gp, gm = np.exp2(G), np.exp2(-G)

    def outputs(q, e, y, p, inv):
        uq, ue, uy = Hm @ y, Dm @ y, Hm.T @ q + Dm.T @ e
        return p * uq, p * Be * ue + inv * uy, p * K * ue, q * uq + e * ue - y * uy

    ref = outputs(Q * gp, Be * K * gp, K * gm, gp, gm)
    for center in (G.mean(0), (G.max(0) + G.min(0)) / 2, G[0], G[-1]):
        a, z = np.exp2(G - center), np.exp2(center - G)
        for x, y in zip(ref, outputs(Q * a, Be * K * a, K * z, a, z)):
            np.testing.assert_allclose(x, y, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("family", ["kda", "gdn2"])
def test_real_captured_intra_fixture(family):
    """The reference's sealed FLA-captured intra inputs (validation/npu950_intra):
    hash check, finiteness with gates x10 (test_npu950_prepared.py:70-78), and the
    pairwise oracle pinned by finite differences of the scalar objective on a
    slice of the real data."""
    meta = json.loads((GOLDEN / "npu950_intra_metadata.json").read_text())[family]
    path = GOLDEN / f"npu950_intra_{family}.npz"
    assert hashlib.sha256(path.read_bytes()).hexdigest() == meta["fixture_sha256"]
    with np.load(path, allow_pickle=False) as data:
        x = {k: data[k].astype(np.float64) for k in data.files}
    assert x["k"].shape == (1, 64, 4, 128)
    vec = family == "gdn2"
    be = x["b"] if vec else x["beta"]
    base = O.intra_pairwise(x["q"], x["k"], x["g"], be, x["dAqk"], x["dAkk"], x["dq"], x["dk"], x["db"], x["dg"],
                            vector_beta=vec)
    assert all(np.isfinite(o).all() for o in base)
    wide = O.intra_pairwise(x["q"], x["k"], x["g"] * 10, be, x["dAqk"], x["dAkk"], x["dq"], x["dk"], x["db"],
                            x["dg"], vector_beta=vec)
    assert all(np.isfinite(o).all() for o in wide)
    # finite-difference pin on head 1, first 16 tokens, first 16 key channels
    sl = (0, slice(0, 16), 1)
    q, k, g = x["q"][sl][:, :16], x["k"][sl][:, :16], x["g"][sl][:, :16] * np.log(2)
    bb = x["b"][sl][:, :16] if vec else x["beta"][sl][:, None]
    l = np.tril(x["dAqk"][sl][:, :16])
    d = np.tril(x["dAkk"][sl][:, :16], -1)
    z = np.zeros((1, 16, 1, 16))
    outs = O.intra_pairwise(q[None, :, None], k[None, :, None], (g / np.log(2))[None, :, None],
                            (bb if vec else bb[:, 0])[None, :, None], l[None, :, None], d[None, :, None],
                            z, z, z if vec else np.zeros((1, 16, 1)), z, vector_beta=vec)
    dq, dk, db, dg = (o[0, :, 0] for o in outs)
    rng = np.random.default_rng(3)
    for i, (inp, grad) in enumerate(zip((q, k, g, bb), (dq, dk, dg, db if vec else db[:, None]))):
        direction = rng.normal(size=inp.shape)
        args = [q, k, g, bb]
        pos, neg = list(args), list(args)
        eps = 1e-6
        pos[i] = inp + eps * direction
        neg[i] = inp - eps * direction
        num = (O.intra_objective(*pos, l, d) - O.intra_objective(*neg, l, d)) / (2 * eps)
        np.testing.assert_allclose(num, np.sum(grad * direction), rtol=1e-6, atol=1e-6)


def test_error_metric_semantics():
    """validation.py:40-45: rel-L2 against the limit, max-abs when the reference vanishes."""
    assert O.error(np.ones(4), np.ones(4) * 1.001, .008)["passed"]
    assert not O.error(np.ones(4), np.ones(4) * 1.1, .008)["passed"]
    assert O.error(np.zeros(4), np.full(4, 1e-7), .008)["passed"]
    assert not O.error(np.zeros(4), np.full(4, 1e-3), .008)["passed"]
    assert not O.error(np.ones(4), np.array([1, 1, np.nan, 1.]), .008)["passed"]


@pytest.mark.parametrize("family", O.FAMILIES)
def test_oracle_reproduces_committed_golden_vectors(family):
    """Regression pin: the committed family vectors (tests/golden/make_golden.py)."""
    from tests.golden.make_golden import load
    ins, outs = load(family)
    n = lambda k: None if k not in ins else ins[k].double().numpy()
    ref = O.backward(family, n("q"), n("k"), n("v"), g=n("g"), beta=n("beta"), b=n("b"), w=n("w"),
                     h0=n("initial_state"), dO=n("dO"), dht=n("dht"))
    for name, expect in outs.items():
        got = ref["fwd"][name] if name in ("o", "final") else ref[name]
        np.testing.assert_allclose(got, expect, rtol=1e-5, atol=1e-6, err_msg=name)
