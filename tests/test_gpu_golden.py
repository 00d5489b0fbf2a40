"""Committed golden vectors through the public optimized operators on the GPU
(reference tolerances, validation.py:40-45,68)."""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests.golden.make_golden import load

pytestmark = pytest.mark.gpu

OPNAME = {"kda": "chunk_kda", "gdn": "chunk_gated_delta_rule", "gdn2": "chunk_gdn2", "delta": "chunk_delta_rule"}
GRAD = {"q": "dq", "k": "dk", "v": "dv", "g": "dg", "beta": "dbeta", "b": "db", "w": "dw", "initial_state": "dh0"}


@pytest.mark.parametrize("op", ["kda", "gdn", "gdn2", "delta"])
def test_golden_family_vectors(op):
    import rewy_amd as fdr
    print(f"\n[golden] op={op}", flush=True)
    ins, outs = load(op)
    dev = torch.device("cuda")
    dO, dht = ins.pop("dO").to(dev), ins.pop("dht").to(dev)
    xg = {k: v.to(dev).requires_grad_() for k, v in ins.items()}
    kw = dict(disable_recompute=True) if op in ("kda", "gdn2") else {}
    fdr.stats(reset=True)
    with fdr.use_backend("optimized"):
        o, ht = getattr(fdr, OPNAME[op])(**xg, output_final_state=True, **kw)
    grads = torch.autograd.grad((o, ht), tuple(xg.values()), (dO, dht))
    torch.cuda.synchronize()
    fdr.assert_used((op,))
    assert O.error(outs["o"], o.detach().float().cpu().numpy(), 0.008)["passed"]
    for (name, _), g in zip(xg.items(), grads):
        e = O.error(outs[GRAD[name]], g.double().cpu().numpy(), O.limit_for(GRAD[name]))
        assert e["passed"], (name, e)
