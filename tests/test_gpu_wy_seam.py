"""KDA's kernel-level WY seam (fdr_chunk_bwd_wy, ``backends.wy.chunk_kda_bwd_wy_dqkg_fused``:
FLA's chunk_kda_bwd_wy_dqkg_fused as the reference replaces its kernel,
backends/backward.py:23-25, kernels/kda_residual_npu_onchip.py:683-702).

* against the fp64 oracle's own terms (oracle/delta_oracle.py ``_post``): dq = the state term
  dq_s, dk = dk_s + beta 2^g E-bar, dv = beta P, dA = D = -strict_tril(P R^T), dg = the
  pre-cumsum dG without the intra terms; rel-L2 1e-2 (fp32 outputs of bf16 products);
* composed as the reference composes its seams -- the WY seam, then the matrix intra
  (``chunk_kda_bwd_intra`` with beta_complete, dAqk = scale tril(dO v_new^T)), then the
  in-chunk reverse cumsum of dg -- against the fused chunk kernel on the same inputs.
"""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests.test_gpu_stages import _np, _rel, _setup

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, seed, gate="default", bz=0):
    from rewy_amd import ops
    xs, dO, sv = _setup("kda", B, T, H, seed=seed, gate=gate, beta_zero_every=bz)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    dh, dR, _ = ops.state_bwd(cu(sv["qg"]), cu(sv["kg"]), cu(sv["w"]), cu(sv["gc"]), 2, cu(dO), sv["scale"],
                              aqk=cu(sv["Aqk"]))
    args = dict(q=cu(xs["q"]), k=cu(xs["k"]), v=cu(xs["v"]), v_new=cu(sv["v_new"]), g=cu(sv["gc"]),
                beta=cu(xs["beta"]), A=cu(sv["Akk"]), h=cu(sv["h"]), do=cu(dO), dh=dh, dv=dR, scale=sv["scale"])
    return xs, dO, sv, args


@pytest.mark.parametrize("shape,gate,bz", [((1, 128, 2), "default", 0), ((2, 192, 2), "wide", 5)])
def test_wy_seam_matches_the_oracle_terms(shape, gate, bz):
    from rewy_amd.backends.wy import chunk_kda_bwd_wy_dqkg_fused
    B, T, H = shape
    print(f"\n[wy] oracle terms shape={shape} gate={gate} beta_zero_every={bz}", flush=True)
    xs, dO, sv, a = _inputs(B, T, H, 91, gate, bz)
    dq, dk, dv, db, dg, dA = chunk_kda_bwd_wy_dqkg_fused(**a)
    torch.cuda.synchronize()
    C = 64
    G = _np(sv["gc"]) * O.LN2
    Q, Kc, Vc, Gc, Ac, dOc, dRc, Rc = (O._to_chunks(x, C) for x in (
        _np(xs["q"]), _np(xs["k"]), _np(xs["v"]), G, _np(sv["Akk"]), _np(dO), _np(a["dv"]), _np(sv["v_new"])))
    Bc = O._to_chunks(_np(xs["beta"])[..., None], C)
    hs = _np(sv["h"]).transpose(0, 2, 1, 3, 4)
    dhs = _np(a["dh"]).transpose(0, 2, 1, 3, 4)
    post = O._post(Q, Kc, Vc, Gc, Bc, np.ones_like(Vc) * Bc, Ac, hs, dhs, Rc, dOc, dRc, a["scale"], C)
    gam = np.exp(Gc)
    P, D = post["P"], post["D"]
    Ebar = -(P @ O._T(hs))
    dq_s = (dOc @ O._T(hs)) * gam * a["scale"]
    dk_s = (Rc @ O._T(dhs)) * np.exp(Gc[..., -1:, :] - Gc)
    dG = Q * dq_s - Kc * dk_s + Bc * Kc * gam * Ebar
    dG[..., -1, :] += gam[..., -1, :] * (hs * dhs).sum(-1) + (Kc * dk_s).sum(-2)
    ref = dict(dq=dq_s, dk=dk_s + Bc * gam * Ebar, dv=Bc * P, dA=D, dg=dG)
    got = dict(dq=dq, dk=dk, dv=dv, dA=dA, dg=dg)
    errs = {n: _rel(_np(got[n]), O._from_chunks(r)) for n, r in ref.items()}
    print("WY seam vs oracle terms", errs, flush=True)
    for n, e in errs.items():
        assert e < 1e-2, (n, errs)


@pytest.mark.parametrize("shape,gate,bz", [((2, 256, 3), "default", 0), ((1, 192, 2), "wide", 4)])
def test_wy_then_intra_equals_the_fused_kernel(shape, gate, bz):
    from rewy_amd import ops
    from rewy_amd.backends.intra import chunk_kda_bwd_intra
    from rewy_amd.backends.wy import chunk_kda_bwd_wy_dqkg_fused
    B, T, H = shape
    print(f"\n[wy] composed shape={shape} gate={gate} beta_zero_every={bz}", flush=True)
    xs, dO, sv, a = _inputs(B, T, H, 92, gate, bz)
    dq, dk, dv, db, dg, dA = chunk_kda_bwd_wy_dqkg_fused(**a)
    # dAqk = scale tril(dO v_new^T) per chunk (FLA's chunk_kda_bwd_dAv output)
    dOc = a["do"].float().view(B, T // 64, 64, H, 128).transpose(2, 3)
    Rc = a["v_new"].float().view(B, T // 64, 64, H, 128).transpose(2, 3)
    dAqk = (a["scale"] * torch.tril(dOc @ Rc.transpose(-1, -2))).transpose(2, 3).reshape(B, T, H, 64).contiguous()
    dq, dk, db, dg = chunk_kda_bwd_intra(a["q"], a["k"], a["g"], a["beta"], dAqk, dA, dq, dk, db, dg,
                                         beta_complete=True)
    dg = dg.view(B, T // 64, 64, H, 128).flip(2).cumsum(2).flip(2).reshape(B, T, H, 128)
    ref = ops.chunk_bwd(a["q"], a["k"], a["v"], a["v_new"], a["do"], a["dv"], a["g"], ops.GATE_VECTOR, a["A"],
                        a["h"], a["dh"], a["scale"], beta=a["beta"])
    torch.cuda.synchronize()
    assert torch.equal(dv, ref["dv"])
    errs = {n: _rel(_np(x), _np(ref[r])) for n, x, r in (("dq", dq, "dq"), ("dk", dk, "dk"), ("dbeta", db, "dbeta"),
                                                        ("dg", dg, "dg"))}
    print("WY + intra vs fused", errs, flush=True)
    for n, e in errs.items():
        assert e < (5e-3 if n in ("dq", "dk") else 1e-4), (n, errs)
