"""The kernel-level seams under FLA's names, with and without cu_seqlens.

* ``backends.state.chunk_gated_delta_rule_bwd_dhu`` (FLA's name; the reference's GDN2
  replacement ``kernels/vector_state_gpu.py:47-67``) against the fp64 oracle's
  ``stage_state_bwd`` for the vector gate (gk, gate-weighted q / k), the scalar gate (g, raw
  q / k) and no gate, K-first and V-first states; with cu_seqlens (a one-token and an empty
  sequence among them) against the same sequences run one at a time as dense rows.
* ``backends.wy.chunk_gdn2_bwd_wy_dqkg_fused`` (the reference's ``gdn2_consumer_fp32.residual``)
  composed with ``backends.intra.chunk_gdn2_bwd_intra`` and the in-chunk reverse cumsum of dg,
  as FLA's chunk_gdn2_bwd composes them, against the fused chunk kernel; and its own terms
  against the oracle's ``_post`` (dv2 = w P, dw = v P, DM = D).
* The KDA WY seam and both intra seams on a packed batch whose sequences start anywhere,
  against the same sequences padded to whole chunks and run as dense rows.
Tolerances: rel-L2 1e-2 for bf16 outputs against the oracle, 5e-3 / 1e-4 for fp32 partial
sums composed in a different order, bit equality where the arithmetic is the same.
"""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests.test_gpu_stages import _np, _rel, _setup

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")


def _cu(x):
    return None if x is None else x.to(DEV).contiguous()


@pytest.mark.parametrize("vf", [False, True])
@pytest.mark.parametrize("op", ["kda", "gdn", "delta"])
def test_state_seam_matches_the_oracle(op, vf):
    from rewy_amd.backends.state import chunk_gated_delta_rule_bwd_dhu
    B, T, H = 2, 192, 2
    print(f"\n[seam state] op={op} state_v_first={vf}", flush=True)
    xs, dO, sv = _setup(op, B, T, H, seed=61)
    gc = sv["gc"]
    dht = torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(4)) * 0.1
    dvl = torch.from_numpy(O.dv_local(_np(sv["Aqk"]), _np(dO))).bfloat16()
    kw = dict(w=_cu(sv["w"]), do=_cu(dO), dv=_cu(dvl), h0=_cu(xs["initial_state"]), scale=sv["scale"],
              dht=_cu(dht.transpose(-1, -2) if vf else dht), state_v_first=vf)
    if op == "kda":
        dh, dh0, dr = chunk_gated_delta_rule_bwd_dhu(_cu(sv["qg"]), _cu(sv["kg"]), gk=_cu(gc), **kw)
        oq, ok_, og = _np(sv["qg"]), _np(sv["kg"]), _np(gc)
    else:
        dh, dh0, dr = chunk_gated_delta_rule_bwd_dhu(_cu(xs["q"]), _cu(xs["k"]), g=_cu(gc), **kw)
        gcn = np.zeros((B, T, H)) if gc is None else _np(gc)
        G = O._to_chunks(gcn[..., None], 64)
        oq = O._from_chunks(O._to_chunks(_np(xs["q"]), 64) * np.exp2(G))
        ok_ = O._from_chunks(O._to_chunks(_np(xs["k"]), 64) * np.exp2(G[..., -1:, :] - G))
        og = np.broadcast_to(gcn[..., None], (B, T, H, 128))
    torch.cuda.synchronize()
    assert dh.dtype == torch.bfloat16 and dh0.dtype == torch.float32 and dr.shape == dvl.shape
    rdh, rdR, rdh0 = O.stage_state_bwd(oq, ok_, _np(sv["w"]), og, _np(dO), _np(dvl), dht=_np(dht),
                                       scale=sv["scale"])
    if vf:
        rdh, rdh0 = rdh.swapaxes(-1, -2), rdh0.swapaxes(-1, -2)
    e = dict(dh=_rel(_np(dh), rdh), dr=_rel(_np(dr), rdR), dh0=_rel(_np(dh0), rdh0))
    print("state seam vs oracle", e, flush=True)
    assert e["dh"] < 1e-2 and e["dr"] < 1e-2 and e["dh0"] < 5e-3, e


def test_state_seam_packed_batch_matches_rows_one_at_a_time():
    from rewy_amd.backends.state import chunk_gated_delta_rule_bwd_dhu
    lens = [100, 0, 64, 1, 230]          # an empty sequence passes its state through
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    Tt, H = int(cu[-1]), 2
    print(f"\n[seam state varlen] lens={lens}", flush=True)
    gen = torch.Generator().manual_seed(62)
    qg = torch.nn.functional.normalize(torch.randn(1, Tt, H, 128, generator=gen), dim=-1).bfloat16()
    kg = torch.nn.functional.normalize(torch.randn(1, Tt, H, 128, generator=gen), dim=-1).bfloat16()
    w = (torch.randn(1, Tt, H, 128, generator=gen) * 0.1).bfloat16()
    do = torch.randn(1, Tt, H, 128, generator=gen).bfloat16()
    dv = torch.randn(1, Tt, H, 128, generator=gen).bfloat16()
    # chunk-local log2 cumsums of a vector gate, restarting at every sequence's chunks
    graw = torch.nn.functional.logsigmoid(torch.randn(1, Tt, H, 128, generator=gen) + 2) / np.log(2)
    gk = torch.empty_like(graw)
    for s in range(len(lens)):
        for c0 in range(int(cu[s]), int(cu[s + 1]), 64):
            c1 = min(c0 + 64, int(cu[s + 1]))
            gk[:, c0:c1] = graw[:, c0:c1].cumsum(1)
    h0 = torch.zeros(len(lens), H, 128, 128)
    dht = torch.randn(len(lens), H, 128, 128, generator=gen) * 0.1
    dh, dh0, dr = chunk_gated_delta_rule_bwd_dhu(_cu(qg), _cu(kg), _cu(w), _cu(do), _cu(dv), gk=_cu(gk), h0=_cu(h0),
                                                 dht=_cu(dht), scale=0.1, cu_seqlens=_cu(cu))
    torch.cuda.synchronize()
    ch = 0
    for s, n in enumerate(lens):
        a, b = int(cu[s]), int(cu[s + 1])
        nc = (n + 63) // 64
        pad = nc * 64 - n
        if n == 0:
            assert torch.equal(dh0[s].cpu(), dht[s]), s
            continue

        def seq(x):
            y = x[:, a:b]
            return torch.cat([y, torch.zeros(1, pad, *y.shape[2:], dtype=y.dtype)], 1) if pad else y
        # padded rows: zero operands and the last real row's gate (the kernels read a missing row so)
        gks = seq(gk)
        if pad:
            gks[:, n:] = gk[:, b - 1:b]
        rdh, rdh0, rdr = chunk_gated_delta_rule_bwd_dhu(_cu(seq(qg)), _cu(seq(kg)), _cu(seq(w)), _cu(seq(do)),
                                                        _cu(seq(dv)), gk=_cu(gks), h0=_cu(h0[s:s + 1]),
                                                        dht=_cu(dht[s:s + 1]), scale=0.1)
        torch.cuda.synchronize()
        e = dict(dh=_rel(_np(dh[:, ch:ch + nc]), _np(rdh)), dh0=_rel(_np(dh0[s:s + 1]), _np(rdh0)),
                 dr=_rel(_np(dr[:, a:b]), _np(rdr[:, :n])))
        print("sequence", s, e, flush=True)
        assert e["dh"] < 1e-5 and e["dh0"] < 1e-5 and e["dr"] < 1e-5, (s, e)
        ch += nc


def _gdn2_inputs(B, T, H, seed):
    from rewy_amd import ops
    xs, dO, sv = _setup("gdn2", B, T, H, seed=seed)
    dh, dR, _ = ops.state_bwd(_cu(sv["qg"]), _cu(sv["kg"]), _cu(sv["w"]), _cu(sv["gc"]), 2, _cu(dO), sv["scale"],
                              aqk=_cu(sv["Aqk"]))
    a = dict(q=_cu(xs["q"]), k=_cu(xs["k"]), v=_cu(xs["v"]), v_new=_cu(sv["v_new"]), g=_cu(sv["gc"]),
             b=_cu(xs["b"]), w_gate=_cu(xs["w"]), A=_cu(sv["Akk"]), h=_cu(sv["h"]), do=_cu(dO), dh=dh, dv=dR,
             scale=sv["scale"])
    return xs, dO, sv, a


def _daqk(a, B, T, H):
    """scale tril(dO v_new^T) per chunk (FLA's dAv output), [B,T,H,64] fp32."""
    dOc = a["do"].float().view(B, T // 64, 64, H, 128).transpose(2, 3)
    Rc = a["v_new"].float().view(B, T // 64, 64, H, 128).transpose(2, 3)
    return (a["scale"] * torch.tril(dOc @ Rc.transpose(-1, -2))).transpose(2, 3).reshape(B, T, H, 64).contiguous()


def test_gdn2_wy_seam_matches_the_oracle_terms():
    from rewy_amd.backends.wy import chunk_gdn2_bwd_wy_dqkg_fused
    B, T, H = 1, 192, 2
    print(f"\n[seam gdn2 wy] oracle terms B={B} T={T} H={H}", flush=True)
    xs, dO, sv, a = _gdn2_inputs(B, T, H, 63)
    dq, dk, dv2, db, dw, dg, dA = chunk_gdn2_bwd_wy_dqkg_fused(**a)
    torch.cuda.synchronize()
    C = 64
    G = _np(sv["gc"]) * O.LN2
    Q, Kc, Vc, Gc, Ac, dOc, dRc, Rc, Bc, Wc = (O._to_chunks(x, C) for x in (
        _np(xs["q"]), _np(xs["k"]), _np(xs["v"]), G, _np(sv["Akk"]), _np(dO), _np(a["dv"]), _np(sv["v_new"]),
        _np(xs["b"]), _np(xs["w"])))
    hs = _np(sv["h"]).transpose(0, 2, 1, 3, 4)
    dhs = _np(a["dh"]).transpose(0, 2, 1, 3, 4)
    post = O._post(Q, Kc, Vc, Gc, Bc, Wc, Ac, hs, dhs, Rc, dOc, dRc, a["scale"], C)
    gam = np.exp(Gc)
    P = post["P"]
    Ebar = -(P @ O._T(hs))
    dq_s = (dOc @ O._T(hs)) * gam * a["scale"]
    dk_s = (Rc @ O._T(dhs)) * np.exp(Gc[..., -1:, :] - Gc)
    dG = Q * dq_s - Kc * dk_s + Bc * Kc * gam * Ebar
    dG[..., -1, :] += gam[..., -1, :] * (hs * dhs).sum(-1) + (Kc * dk_s).sum(-2)
    ref = dict(dq=dq_s, dk=dk_s + Bc * gam * Ebar, dv=post["dv"], dw=post["dw"], db=Kc * gam * Ebar, dA=post["D"],
               dg=dG)
    got = dict(dq=dq, dk=dk, dv=dv2, dw=dw, db=db, dA=dA, dg=dg)
    errs = {n: _rel(_np(got[n]), O._from_chunks(r)) for n, r in ref.items()}
    print("GDN2 WY seam vs oracle terms", errs, flush=True)
    for n, e in errs.items():
        assert e < 1e-2, (n, errs)


@pytest.mark.parametrize("vf", [False, True])
def test_gdn2_wy_then_intra_equals_the_fused_kernel(vf):
    from rewy_amd import ops
    from rewy_amd.backends.intra import chunk_gdn2_bwd_intra
    from rewy_amd.backends.wy import chunk_gdn2_bwd_wy_dqkg_fused
    B, T, H = 2, 256, 3
    print(f"\n[seam gdn2 wy+intra] B={B} T={T} H={H} state_v_first={vf}", flush=True)
    xs, dO, sv, a = _gdn2_inputs(B, T, H, 64)
    ref = ops.chunk_bwd(a["q"], a["k"], a["v"], a["v_new"], a["do"], a["dv"], a["g"], ops.GATE_VECTOR, a["A"],
                        a["h"], a["dh"], a["scale"], b=a["b"], w=a["w_gate"])
    if vf:
        # FLA's V-first per-chunk states, as FLA's chunk_gdn2_bwd hands them over
        a = dict(a, h=a["h"].transpose(-1, -2).contiguous(), dh=a["dh"].transpose(-1, -2).contiguous())
    dq, dk, dv2, db, dw, dg, dA = chunk_gdn2_bwd_wy_dqkg_fused(**a, state_v_first=vf)
    dq, dk, db, dg = chunk_gdn2_bwd_intra(a["q"], a["k"], a["g"], a["b"], _daqk(a, B, T, H), dA, dq, dk, db, dg)
    dg = dg.view(B, T // 64, 64, H, 128).flip(2).cumsum(2).flip(2).reshape(B, T, H, 128)
    torch.cuda.synchronize()
    assert torch.equal(dv2, ref["dv"]) and torch.equal(dw, ref["dw"])
    errs = {n: _rel(_np(x), _np(ref[n])) for n, x in (("dq", dq), ("dk", dk), ("db", db), ("dg", dg))}
    print("GDN2 WY + intra vs fused", errs, flush=True)
    for n, e in errs.items():
        assert e < (5e-3 if n in ("dq", "dk", "db") else 1e-4), (n, errs)


def _packed_and_padded(op, lens, H, seed):
    """Inputs of the chunk stage for a packed batch (sequences starting anywhere) and the same
    sequences each padded to whole chunks as rows of a dense batch (zero operands, the gate's
    last real row repeated), from one dense forward over the padded rows."""
    from rewy_amd import ops
    nch = [(n + 63) // 64 for n in lens]
    Tp = 64 * max(nch)
    Bp = len(lens)
    xs, dO, sv = _setup(op, Bp, Tp, H, seed=seed)
    # zero the padding (every sequence ends at its length), then re-run the forward on it
    from rewy_amd.forward import chunk_forward
    for s, n in enumerate(lens):
        for name in ("q", "k", "v", "b", "w"):
            if name in xs:
                xs[name][s, n:] = 0
        if "beta" in xs:
            xs["beta"][s, n:] = 0
        xs["g"][s, n:] = 0
        dO[s, n:] = 0
    _, _, sv = chunk_forward(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"), b=xs.get("b"),
                             w=xs.get("w"), initial_state=xs.get("initial_state"))
    dev = {n: _cu(x) for n, x in list(xs.items()) + [("dO", dO)] + [(f"sv_{n}", v) for n, v in sv.items()
                                                                       if torch.is_tensor(v)]}
    dh, dR, _ = ops.state_bwd(dev["sv_qg"], dev["sv_kg"], dev["sv_w"], dev["sv_gc"], 2, dev["dO"], sv["scale"],
                              aqk=dev["sv_Aqk"])
    dev["dh"], dev["dR"] = dh, dR
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)

    def pack(x):      # [Bp, Tp, ...] token rows -> [1, sum(lens), ...]
        return torch.cat([x[s:s + 1, :n] for s, n in enumerate(lens)], 1).contiguous()

    def pack_chunks(x):     # [Bp, NTp, ...] per-chunk states -> [1, sum(nch), ...]
        return torch.cat([x[s:s + 1, :c] for s, c in enumerate(nch)], 1).contiguous()
    return dev, sv["scale"], cu, pack, pack_chunks


@pytest.mark.parametrize("op", ["kda", "gdn2"])
def test_wy_and_intra_seams_on_a_packed_batch(op):
    from rewy_amd.backends.intra import chunk_gdn2_bwd_intra, chunk_kda_bwd_intra
    from rewy_amd.backends.wy import chunk_gdn2_bwd_wy_dqkg_fused, chunk_kda_bwd_wy_dqkg_fused
    lens, H = [150, 64, 0, 37, 1, 200], 2
    print(f"\n[seam varlen] op={op} lens={lens}", flush=True)
    d, scale, cu, pack, pack_chunks = _packed_and_padded(op, lens, H, 65)
    Bp, Tp = d["q"].shape[:2]
    common = dict(q=d["q"], k=d["k"], v=d["v"], v_new=d["sv_v_new"], g=d["sv_gc"], A=d["sv_Akk"], h=d["sv_h"],
                  do=d["dO"], dh=d["dh"], dv=d["dR"], scale=scale)
    if op == "kda":
        dense = chunk_kda_bwd_wy_dqkg_fused(beta=d["beta"], **common)
    else:
        dense = chunk_gdn2_bwd_wy_dqkg_fused(b=d["b"], w_gate=d["w"], **common)
    dAqk = _daqk(dict(do=d["dO"], v_new=d["sv_v_new"], scale=scale), Bp, Tp, H)
    packed_in = {n: (pack_chunks(x) if n in ("h", "dh") else pack(x)) if torch.is_tensor(x) else x
                 for n, x in common.items()}
    cuc = _cu(cu)
    if op == "kda":
        got = chunk_kda_bwd_wy_dqkg_fused(beta=pack(d["beta"]), cu_seqlens=cuc, **packed_in)
    else:
        got = chunk_gdn2_bwd_wy_dqkg_fused(b=pack(d["b"]), w_gate=pack(d["w"]), cu_seqlens=cuc, **packed_in)
    torch.cuda.synchronize()
    names = ("dq", "dk", "dv", "db", "dg", "dA") if op == "kda" else ("dq", "dk", "dv", "db", "dw", "dg", "dA")
    for n, x, r in zip(names, got, dense):
        assert torch.equal(x, pack(r)), (op, "WY seam", n)
    # the intra seam on the packed batch against the padded rows
    ga, gb = [x.clone() for x in got], [x.clone() for x in dense]
    iq = dict(zip(names, ga))
    rq = dict(zip(names, gb))
    if op == "kda":
        chunk_kda_bwd_intra(packed_in["q"], packed_in["k"], packed_in["g"], pack(d["beta"]), pack(dAqk), iq["dA"],
                            iq["dq"], iq["dk"], iq["db"], iq["dg"], cu_seqlens=cuc, beta_complete=True)
        chunk_kda_bwd_intra(d["q"], d["k"], d["sv_gc"], d["beta"], dAqk, rq["dA"], rq["dq"], rq["dk"], rq["db"],
                            rq["dg"], beta_complete=True)
    else:
        chunk_gdn2_bwd_intra(packed_in["q"], packed_in["k"], packed_in["g"], pack(d["b"]), pack(dAqk), iq["dA"],
                             iq["dq"], iq["dk"], iq["db"], iq["dg"], cu_seqlens=cuc)
        chunk_gdn2_bwd_intra(d["q"], d["k"], d["sv_gc"], d["b"], dAqk, rq["dA"], rq["dq"], rq["dk"], rq["db"],
                             rq["dg"])
    torch.cuda.synchronize()
    for n in ("dq", "dk", "db", "dg"):
        assert torch.equal(iq[n], pack(rq[n])), (op, "intra seam", n)
