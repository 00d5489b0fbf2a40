"""Parity of the affine-step recurrences (fdr_affine_prep_bwd / _prep_fwd / _scan /
_side) with the fp64 oracle's stage functions, and with the direct kernels
(fdr_state_bwd, fdr_fwd_h) on the same inputs.

Cases cover every gate mode, chunk counts that are and are not multiples of the
scan's prefetch depth (4), one-chunk sequences, every value-block width, a
precomputed dv_local in place of Aqk, and a zero / non-zero initial state.
Tolerances as for the direct kernels: rel-L2 1e-2 for bf16 outputs, 5e-3 for fp32.
"""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests.test_gpu_stages import GATE, _np, _rel, _setup

pytestmark = pytest.mark.gpu

BWD_CASES = [
    ("kda", (1, 64 * 9, 2), 16, "aqk"),
    ("gdn", (2, 64 * 6, 1), 16, "aqk"),
    ("delta", (1, 64 * 5, 3), 32, "aqk"),
    ("gdn2", (1, 64 * 8, 2), 64, "aqk"),
    ("kda", (1, 64, 2), 16, "dv"),
    ("gdn", (1, 64 * 3, 2), 32, "dv"),
]


def _gated(op, xs, sv, B, T, H):
    """Inputs of the state recurrence as both paths take them, and the fp64 oracle's."""
    gc = sv["gc"]
    if op in ("kda", "gdn2"):
        qs, ks = sv["qg"], sv["kg"]
        return qs, ks, _np(qs), _np(ks), _np(gc)
    qs, ks = xs["q"], xs["k"]
    gcn = np.zeros((B, T, H)) if gc is None else _np(gc)
    G = O._to_chunks(gcn[..., None], 64)
    oq = O._from_chunks(O._to_chunks(_np(xs["q"]), 64) * np.exp2(G))
    ok_ = O._from_chunks(O._to_chunks(_np(xs["k"]), 64) * np.exp2(G[..., -1:, :] - G))
    return qs, ks, oq, ok_, np.broadcast_to(gcn[..., None], (B, T, H, 128))


@pytest.mark.parametrize("op,shape,vb,dv_from", BWD_CASES)
def test_affine_state_bwd(op, shape, vb, dv_from):
    from rewy_amd import ops
    B, T, H = shape
    print(f"\n[affine bwd] op={op} B={B} T={T} H={H} value_block={vb} dv={dv_from}", flush=True)
    xs, dO, sv = _setup(op, B, T, H, seed=23)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    scale = sv["scale"]
    qs, ks, oq, ok_, og = _gated(op, xs, sv, B, T, H)
    odv = O.dv_local(_np(sv["Aqk"]), _np(dO))
    dht = torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(5)) * 0.1
    kw = dict(aqk=cu(sv["Aqk"])) if dv_from == "aqk" else dict(dv=cu(torch.from_numpy(odv).bfloat16()))
    args = (cu(qs), cu(ks), cu(sv["w"]), cu(sv["gc"]), GATE[op], cu(dO), scale)
    dh, dR, dh0 = ops.state_bwd(*args, dht=cu(dht), value_block=vb, method="affine", **kw)
    ddh, ddR, ddh0 = ops.state_bwd(*args, dht=cu(dht), method="direct", **kw)
    torch.cuda.synchronize()
    odv_in = odv if dv_from == "aqk" else _np(kw["dv"])
    rdh, rdR, rdh0 = O.stage_state_bwd(oq, ok_, _np(sv["w"]), og, _np(dO), odv_in, dht=_np(dht), scale=scale)
    e = dict(dh=_rel(_np(dh), rdh), dR=_rel(_np(dR), rdR), dh0=_rel(_np(dh0), rdh0))
    d = dict(dh=_rel(_np(dh), _np(ddh)), dR=_rel(_np(dR), _np(ddR)), dh0=_rel(_np(dh0), _np(ddh0)))
    print("vs oracle", e, "vs direct", d, flush=True)
    assert e["dh"] < 1e-2 and e["dR"] < 1e-2 and e["dh0"] < 5e-3, e
    assert d["dh"] < 1e-2 and d["dR"] < 1e-2 and d["dh0"] < 5e-3, d


FWD_CASES = [("kda", (1, 64 * 9, 2), 16), ("gdn", (2, 64 * 6, 1), 32), ("delta", (1, 64 * 5, 3), 64),
             ("gdn2", (1, 64, 2), 16), ("gdn", (1, 64 * 4, 2), 16)]


@pytest.mark.parametrize("op,shape,vb", FWD_CASES)
def test_affine_fwd_h(op, shape, vb):
    from rewy_amd import ops
    from rewy_amd.forward import chunk_forward
    from tests._inputs import make_inputs
    B, T, H = shape
    print(f"\n[affine fwd] op={op} B={B} T={T} H={H} value_block={vb}", flush=True)
    xs, _ = make_inputs(op, B, T, H, seed=29)
    _, _, sv = chunk_forward(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"),
                             b=xs.get("b"), w=xs.get("w"), initial_state=xs["initial_state"],
                             output_final_state=True)
    n = lambda x: None if x is None else x.double().numpy()
    ref = O.forward(op, n(xs["q"]), n(xs["k"]), n(xs["v"]), g=n(xs.get("g")), beta=n(xs.get("beta")),
                    b=n(xs.get("b")), w=n(xs.get("w")), h0=n(xs["initial_state"]))
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    vec = op in ("kda", "gdn2")
    kin = sv["kg"] if vec else xs["k"]
    args = (cu(kin), cu(sv["w"]), cu(sv["u"]), cu(sv["gc"]), GATE[op])
    h, vnew, ht = ops.fwd_h(*args, h0=cu(xs.get("initial_state")), want_final=True, value_block=vb, method="affine")
    dh_, dvn, dht_ = ops.fwd_h(*args, h0=cu(xs.get("initial_state")), want_final=True, method="direct")
    torch.cuda.synchronize()
    e = dict(h=_rel(n(h.cpu()), ref["h"]), v_new=_rel(n(vnew.cpu()), ref["v_new"]),
             final=_rel(n(ht.cpu()), ref["final"]))
    d = dict(h=_rel(n(h.cpu()), n(dh_.cpu())), v_new=_rel(n(vnew.cpu()), n(dvn.cpu())),
             final=_rel(n(ht.cpu()), n(dht_.cpu())))
    print("vs oracle", e, "vs direct", d, flush=True)
    for name in e:
        assert e[name] < 1e-2 and d[name] < 1e-2, (name, e, d)


@pytest.mark.parametrize("op", ["gdn", "delta", "kda", "gdn2"])
def test_affine_recurrences_pair(op):
    """ops.recurrences (both recurrences in one scan launch) against fdr_fwd_h + fdr_state_bwd."""
    from rewy_amd import ops
    B, T, H = 1, 64 * 10, 3
    print(f"\n[affine pair] op={op} B={B} T={T} H={H}", flush=True)
    xs, dO, sv = _setup(op, B, T, H, seed=31)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    qs, ks, *_ = _gated(op, xs, sv, B, T, H)
    g = cu(sv["gc"])
    dht = (torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(7)) * 0.1).to(dev)
    h0 = cu(xs.get("initial_state"))
    args = (cu(qs), cu(ks), cu(sv["w"]))
    got = ops.recurrences(*args, cu(sv["u"]), g, GATE[op], cu(dO), sv["scale"], aqk=cu(sv["Aqk"]), h0=h0, dht=dht)
    h, vnew, _ = ops.fwd_h(cu(ks), cu(sv["w"]), cu(sv["u"]), g, GATE[op], h0=h0, method="direct")
    dh, dR, dh0 = ops.state_bwd(*args, g, GATE[op], cu(dO), sv["scale"], aqk=cu(sv["Aqk"]), dht=dht,
                                method="direct")
    torch.cuda.synchronize()
    e = {n: _rel(_np(a), _np(r)) for n, a, r in zip(("h", "v_new", "dh", "dR", "dh0"), got, (h, vnew, dh, dR, dh0))}
    print("pair vs direct", e, flush=True)
    for n, v in e.items():
        assert v < 1e-2, (n, e)


@pytest.mark.parametrize("op", ["gdn", "kda"])
def test_backend_switches_to_affine_with_same_gradients(op, monkeypatch):
    """The backend's automatic choice (affine at B*H <= 16, >= 8 chunks) gives the
    gradients the direct kernels give; the recompute policy for KDA."""
    from rewy_amd import ops
    from rewy_amd.backends import backward as bw
    B, T, H = 1, 64 * 12, 2
    print(f"\n[affine backend] op={op} B={B} T={T} H={H}", flush=True)
    xs, dO, sv = _setup(op, B, T, H, seed=37)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()

    def run():
        if op == "gdn":
            return bw.gdn_backward(q=cu(xs["q"]), k=cu(xs["k"]), v=cu(xs["v"]), g=cu(sv["gc"]), beta=cu(xs["beta"]),
                                   A=cu(sv["Akk"]), scale=sv["scale"], initial_state=cu(xs.get("initial_state")),
                                   do=cu(dO), dht=None)
        return bw.kda_backward(q=cu(xs["q"]), k=cu(xs["k"]), v=cu(xs["v"]), beta=cu(xs["beta"]), Aqk=cu(sv["Aqk"]),
                               Akk=cu(sv["Akk"]), scale=sv["scale"], initial_state=cu(xs.get("initial_state")),
                               do=cu(dO), dht=None, g=cu(sv["gc"]))
    assert ops.affine_pays(cu(xs["q"]))
    got = run()
    monkeypatch.setattr(ops, "AFFINE_MAX_BH", -1)
    ref = run()
    torch.cuda.synchronize()
    for i, (a, r) in enumerate(zip(got, ref)):
        if torch.is_tensor(r):
            e = _rel(_np(a), _np(r))
            print(i, e, flush=True)
            assert e < 1e-2, (i, e)
