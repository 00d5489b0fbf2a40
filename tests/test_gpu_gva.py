"""Grouped value heads (FLA's GVA: q / k with H heads, v, g, beta and the state with
HV = G * H; reference _compat/kda.py:246-247, _compat/gdn.py:297-298, head map
i_h = i_hv // G) handled by the kernels themselves.

* kernel level: every entry point that reads raw q / k, given q / k with H heads, must
  produce exactly (bit for bit) what it produces when q / k are repeated to HV heads --
  the same arithmetic on the same values (forward prepare, w/u recompute, forward scan,
  output, state recurrence, chunk kernel, standalone intra);
* end to end: the public operators (KDA full saving and recompute, GDN, DeltaNet)
  against the fp64 oracle on repeated q / k (whose dq / dk are then summed over each
  group) at the reference's tolerances, and against the original backend.
"""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu

OPNAME = {"kda": "chunk_kda", "gdn": "chunk_gated_delta_rule", "delta": "chunk_delta_rule"}
GATE = {"delta": 0, "gdn": 1, "kda": 2}
G = 2


def _rep(x):
    return x.repeat_interleave(G, dim=2).contiguous()


def _gva_inputs(op, B, T, HV, seed):
    xs, dO = make_inputs(op, B, T, HV, seed=seed)
    xs["q"] = xs["q"][:, :, ::G].contiguous()
    xs["k"] = xs["k"][:, :, 1::G].contiguous()
    return xs, dO


def _eq(a, b, name):
    assert a.shape == b.shape, (name, a.shape, b.shape)
    assert torch.equal(a, b), (name, float((a.float() - b.float()).abs().max()))


@pytest.mark.parametrize("op", ["kda", "gdn", "delta"])
def test_kernels_map_value_heads_to_qk_heads(op):
    from rewy_amd import ops
    from rewy_amd.hip_forward import GATE_MODE
    B, T, HV = 2, 192, 4
    print(f"\n[gva] kernels op={op}", flush=True)
    xs, dO = _gva_inputs(op, B, T, HV, seed=61)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    q, k, v, beta, g, dO = cu(xs["q"]), cu(xs["k"]), cu(xs["v"]), cu(xs["beta"]), cu(xs.get("g")), cu(dO)
    qr, kr = _rep(q), _rep(k)
    gm = GATE_MODE[op]
    scale = 128 ** -0.5
    # forward: prepare, w/u, scan, output
    gc, Aqk, Akk = ops.fwd_prepare(q, k, g, gm, beta=beta, scale=scale)
    rgc, rAqk, rAkk = ops.fwd_prepare(qr, kr, g, gm, beta=beta, scale=scale)
    for n, a, b in (("gc", gc, rgc), ("Aqk", Aqk, rAqk), ("Akk", Akk, rAkk)):
        if a is not None:
            _eq(a, b, n)
    vec = gm == ops.GATE_VECTOR
    wu = ops.prepare_wu(k, v, Akk, gm, g=gc, beta=beta, q=q, want_qkg=vec, want_aqk=not vec, scale=scale)
    rwu = ops.prepare_wu(kr, v, Akk, gm, g=gc, beta=beta, q=qr, want_qkg=vec, want_aqk=not vec, scale=scale)
    for n in wu:
        if wu[n] is not None:
            _eq(wu[n], rwu[n], n)
    h0 = cu(xs["initial_state"])
    kin, rkin = (wu["kg"], wu["kg"]) if vec else (k, kr)
    h, vn, ht = ops.fwd_h(kin, wu["w"], wu["u"], gc, gm, h0=h0, want_final=True, method="direct")
    rh, rvn, rht = ops.fwd_h(rkin, wu["w"], wu["u"], gc, gm, h0=h0, want_final=True, method="direct")
    for n, a, b in (("h", h, rh), ("v_new", vn, rvn), ("final", ht, rht)):
        _eq(a, b, n)
    aqk = Aqk if vec else wu["Aqk"]
    o = ops.fwd_o(q, gc, gm, Aqk, h, vn, scale)
    _eq(o, ops.fwd_o(qr, gc, gm, Aqk, h, vn, scale), "o")
    # backward: state recurrence (raw q / k for scalar gates), chunk kernel
    qs, ks = (wu["qg"], wu["kg"]) if vec else (q, k)
    rqs, rks = (wu["qg"], wu["kg"]) if vec else (qr, kr)
    dh, dR, dh0 = ops.state_bwd(qs, ks, wu["w"], gc, gm, dO, scale, aqk=aqk, method="direct")
    rdh, rdR, rdh0 = ops.state_bwd(rqs, rks, wu["w"], gc, gm, dO, scale, aqk=aqk, method="direct")
    for n, a, b in (("dh", dh, rdh), ("dR", dR, rdR), ("dh0", dh0, rdh0)):
        _eq(a, b, n)
    out = ops.chunk_bwd(q, k, v, vn, dO, dR, gc, gm, Akk, h, dh, scale, beta=beta)
    ref = ops.chunk_bwd(qr, kr, v, vn, dO, dR, gc, gm, Akk, h, dh, scale, beta=beta)
    torch.cuda.synchronize()
    for n in out:
        if out[n] is not None:
            _eq(out[n], ref[n], n)
    if vec:
        gen = torch.Generator().manual_seed(3)
        dAqk = (torch.randn(B, T, HV, 64, generator=gen) * 0.1).to(dev)
        dAkk = (torch.randn(B, T, HV, 64, generator=gen) * 0.1).to(dev)
        parts = [torch.randn(B, T, HV, 128, generator=gen).to(dev) for _ in range(3)]
        db = torch.randn(B, T, HV, generator=gen).to(dev)
        a = ops.matrix_intra(q, k, gc, dAqk, dAkk, *(x.clone() for x in parts[:2]), db.clone(), parts[2].clone(),
                             beta=beta)
        r = ops.matrix_intra(qr, kr, gc, dAqk, dAkk, *(x.clone() for x in parts[:2]), db.clone(), parts[2].clone(),
                             beta=beta)
        torch.cuda.synchronize()
        for i, (x, y) in enumerate(zip(a, r)):
            if i == 2:
                # db sums the 8 waves' row partials with LDS atomics: order-dependent rounding
                assert torch.allclose(x, y, rtol=1e-6, atol=1e-6), float((x - y).abs().max())
            else:
                _eq(x, y, f"intra {i}")


@pytest.mark.parametrize("op,kw", [("kda", dict(disable_recompute=True)), ("kda", dict(disable_recompute=False)),
                                   ("gdn", {}), ("delta", {})])
def test_public_operators_with_grouped_value_heads(op, kw):
    import rewy_amd as fdr
    print(f"\n[gva] public op={op} kw={kw}", flush=True)
    B, T, HV = 1, 192, 4
    xs, dO = _gva_inputs(op, B, T, HV, seed=62)
    dev = torch.device("cuda")
    dht = torch.randn(B, HV, 128, 128, generator=torch.Generator().manual_seed(8)) * 0.1
    res = {}
    for backend in ("optimized", "original"):
        fdr.stats(reset=True)
        xg = {n: v.to(dev).requires_grad_() for n, v in xs.items()}
        with fdr.use_backend(backend, ops=(op,)):
            o, ht = getattr(fdr, OPNAME[op])(**xg, output_final_state=True, **kw)
        grads = torch.autograd.grad((o, ht), tuple(xg.values()), (dO.to(dev), dht.to(dev)))
        torch.cuda.synchronize()
        res[backend] = dict(zip(xs, grads), o=o, final=ht)
        if backend == "optimized":
            fdr.assert_used((op,))
            assert not any("fallback" in k or "rejected" in k for k in fdr.stats())
    n = lambda x: None if x is None else x.detach().double().cpu().numpy()
    ref = O.backward(op, n(_rep(xs["q"])), n(_rep(xs["k"])), n(xs["v"]), g=n(xs.get("g")), beta=n(xs.get("beta")),
                     h0=n(xs["initial_state"]), dO=n(dO), dht=n(dht))
    gsum = lambda x: x.reshape(B, T, HV // G, G, 128).sum(3)
    ref["dq"], ref["dk"] = gsum(ref["dq"]), gsum(ref["dk"])
    grad = {"q": "dq", "k": "dk", "v": "dv", "g": "dg", "beta": "dbeta", "initial_state": "dh0"}
    for name, r in grad.items():
        if name not in xs:
            continue
        got = n(res["optimized"][name])
        e = O.error(ref[r], got, O.limit_for(r))
        eo = O.error(n(res["original"][name]), got, O.limit_for(r))
        print(f"  {name}: vs oracle {e['relative_l2']:.2e}, vs original {eo['relative_l2']:.2e}", flush=True)
        assert e["passed"] and eo["passed"], (name, e, eo)
    for name in ("o", "final"):
        eo = O.error(n(res["original"][name]), n(res["optimized"][name]), 0.008)
        assert eo["passed"], (name, eo)
