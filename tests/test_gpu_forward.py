"""Parity of the HIP forward (rewy_amd.hip_forward: fdr_fwd_prepare, fdr_prepare_wu,
fdr_fwd_h, fdr_fwd_o) with the fp64 oracle's forward, all four families.

Tolerances (rel-L2): gc 1e-6 and Aqk / Akk 2e-4 (fp32 outputs; the products are
fp32-faithful bf16 hi + lo MFMAs and the inverse is an fp32 block substitution);
bf16 outputs (o, w, u, v_new, h, qg, kg) 1e-2; the fp32 final state 1e-2 (it is
accumulated from bf16 v_new as in FLA).
"""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu


def _rel(a, r):
    a, r = np.asarray(a, np.float64), np.asarray(r, np.float64)
    return float(np.linalg.norm(a - r) / max(np.linalg.norm(r), 1e-30))


CASES = [(op, shp, "default") for op in ("kda", "gdn", "delta", "gdn2") for shp in ((1, 128, 2), (2, 256, 3))]
CASES += [("kda", (1, 192, 2), "wide"), ("gdn2", (1, 128, 2), "wide")]


@pytest.mark.parametrize("op,shape,gate", CASES)
def test_hip_forward_matches_oracle(op, shape, gate):
    from rewy_amd.hip_forward import chunk_forward_hip
    B, T, H = shape
    print(f"\n[forward] op={op} B={B} T={T} H={H} gate={gate}", flush=True)
    xs, _ = make_inputs(op, B, T, H, seed=23, gate=gate)
    n = lambda x: None if x is None else x.double().cpu().numpy()
    ref = O.forward(op, n(xs["q"]), n(xs["k"]), n(xs["v"]), g=n(xs.get("g")), beta=n(xs.get("beta")),
                    b=n(xs.get("b")), w=n(xs.get("w")), h0=n(xs["initial_state"]))
    cu = lambda x: None if x is None else x.cuda()
    o, final, sv = chunk_forward_hip(op, cu(xs["q"]), cu(xs["k"]), cu(xs["v"]), g=cu(xs.get("g")),
                                     beta=cu(xs.get("beta")), b=cu(xs.get("b")), w=cu(xs.get("w")),
                                     initial_state=cu(xs["initial_state"]), output_final_state=True)
    torch.cuda.synchronize()
    errs = dict(o=_rel(n(o), ref["o"]), final=_rel(n(final), ref["final"]), Aqk=_rel(n(sv["Aqk"]), ref["Aqk"]),
                Akk=_rel(n(sv["Akk"]), ref["Akk"]), w=_rel(n(sv["w"]), ref["w"]), u=_rel(n(sv["u"]), ref["u"]),
                v_new=_rel(n(sv["v_new"]), ref["v_new"]), h=_rel(n(sv["h"]), ref["h"]))
    if op != "delta":
        errs["gc"] = _rel(n(sv["gc"]), ref["gc"][..., 0] if op == "gdn" else ref["gc"])
    if op in ("kda", "gdn2"):
        errs.update(qg=_rel(n(sv["qg"]), ref["qg"]), kg=_rel(n(sv["kg"]), ref["kg"]))
    print("rel-L2 vs oracle", {k_: f"{v_:.2e}" for k_, v_ in errs.items()}, flush=True)
    tol = dict(gc=1e-6, Aqk=2e-4, Akk=2e-4)
    for name, e in errs.items():
        assert e <= tol.get(name, 1e-2), (name, errs)
