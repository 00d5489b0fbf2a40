"""Parity of the recompute kernels (fdr_prepare_wu, fdr_fwd_h) with the fp64
oracle's forward intermediates (FLA recompute_w_u_fwd / chunk_gated_delta_rule_fwd_h)."""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu
GATE = {"delta": 0, "gdn": 1, "kda": 2, "gdn2": 2}


def _rel(a, r):
    a, r = np.asarray(a, np.float64), np.asarray(r, np.float64)
    return float(np.linalg.norm(a - r) / max(np.linalg.norm(r), 1e-30))


@pytest.mark.parametrize("op", ["kda", "gdn", "delta", "gdn2"])
@pytest.mark.parametrize("B,T,H", [(1, 128, 2), (2, 256, 3)])
def test_prepare_wu_and_fwd_h(op, B, T, H):
    from rewy_amd import ops
    from rewy_amd.forward import chunk_forward
    print(f"\n[recompute] op={op} B={B} T={T} H={H}", flush=True)
    xs, _ = make_inputs(op, B, T, H, seed=17)
    _, fin, sv = chunk_forward(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"),
                               b=xs.get("b"), w=xs.get("w"), initial_state=xs["initial_state"],
                               output_final_state=True)
    n = lambda x: None if x is None else x.double().numpy()
    ref = O.forward(op, n(xs["q"]), n(xs["k"]), n(xs["v"]), g=n(xs.get("g")), beta=n(xs.get("beta")),
                    b=n(xs.get("b")), w=n(xs.get("w")), h0=n(xs["initial_state"]))
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    vec = op in ("kda", "gdn2")
    pre = ops.prepare_wu(cu(xs["k"]), cu(xs["v"]), cu(sv["Akk"]), GATE[op], g=cu(sv["gc"]),
                         beta=cu(xs.get("beta")), b=cu(xs.get("b")), w=cu(xs.get("w")), q=cu(xs["q"]),
                         want_qkg=vec, want_aqk=not vec, scale=sv["scale"])
    torch.cuda.synchronize()
    errs = dict(w=_rel(n(pre["w"].cpu()), ref["w"]), u=_rel(n(pre["u"].cpu()), ref["u"]))
    if vec:
        errs.update(qg=_rel(n(pre["qg"].cpu()), ref["qg"]), kg=_rel(n(pre["kg"].cpu()), ref["kg"]))
    else:
        errs["Aqk"] = _rel(n(pre["Aqk"].cpu()), ref["Aqk"])
    kin = pre["kg"] if vec else cu(xs["k"])
    h, vnew, ht = ops.fwd_h(kin, pre["w"], pre["u"], cu(sv["gc"]), GATE[op], h0=cu(xs["initial_state"]),
                            want_final=True)
    torch.cuda.synchronize()
    errs.update(h=_rel(n(h.cpu()), ref["h"]), v_new=_rel(n(vnew.cpu()), ref["v_new"]),
                final=_rel(n(ht.cpu()), ref["final"]))
    print("rel-L2 vs oracle", errs, flush=True)
    for name, e in errs.items():
        assert e < (5e-4 if name == "Aqk" else 1e-2), (name, errs)


@pytest.mark.parametrize("op", ["kda", "gdn"])
@pytest.mark.parametrize("vb", [16, 32, 64])
def test_fwd_h_value_blocks(op, vb):
    """Every value-tile width of the direct forward scan against the oracle."""
    from rewy_amd import ops
    from rewy_amd.forward import chunk_forward
    B, T, H = 1, 256, 2
    print(f"\n[fwd_h vb] op={op} value_block={vb}", flush=True)
    xs, _ = make_inputs(op, B, T, H, seed=43)
    _, _, sv = chunk_forward(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"),
                             initial_state=xs["initial_state"], output_final_state=True)
    n = lambda x: None if x is None else x.double().numpy()
    ref = O.forward(op, n(xs["q"]), n(xs["k"]), n(xs["v"]), g=n(xs.get("g")), beta=n(xs.get("beta")),
                    h0=n(xs["initial_state"]))
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    kin = sv["kg"] if op == "kda" else xs["k"]
    h, vnew, ht = ops.fwd_h(cu(kin), cu(sv["w"]), cu(sv["u"]), cu(sv["gc"]), GATE[op], h0=cu(xs["initial_state"]),
                            want_final=True, value_block=vb, method="direct")
    torch.cuda.synchronize()
    errs = dict(h=_rel(n(h.cpu()), ref["h"]), v_new=_rel(n(vnew.cpu()), ref["v_new"]),
                final=_rel(n(ht.cpu()), ref["final"]))
    print("rel-L2 vs oracle", errs, flush=True)
    for name, e in errs.items():
        assert e < 1e-2, (name, errs)
