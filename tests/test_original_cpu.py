"""The PyTorch original-formulation backend (the same-GPU comparator) checked on
the CPU against the fp64 oracle through the public autograd surface."""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests._inputs import make_inputs

OPNAME = {"kda": "chunk_kda", "gdn": "chunk_gated_delta_rule", "gdn2": "chunk_gdn2", "delta": "chunk_delta_rule"}
GRAD = {"q": "dq", "k": "dk", "v": "dv", "g": "dg", "beta": "dbeta", "b": "db", "w": "dw", "initial_state": "dh0"}


@pytest.mark.parametrize("op", ["kda", "gdn", "gdn2", "delta"])
@pytest.mark.parametrize("T", [128, 100])
def test_original_backend_gradients(op, T):
    import rewy_amd as fdr
    xs, dO = make_inputs(op, 1, T, 2, seed=13, beta_zero_every=5 if op != "gdn2" else 0)
    xg = {k: v.clone().requires_grad_() for k, v in xs.items()}
    kw = dict(disable_recompute=True) if op in ("kda", "gdn2") else {}
    with fdr.use_backend("original"):
        o, ht = getattr(fdr, OPNAME[op])(**xg, output_final_state=True, **kw)
    dht = torch.randn(ht.shape, generator=torch.Generator().manual_seed(1)) * 0.1
    grads = torch.autograd.grad((o, ht), tuple(xg.values()), (dO, dht))
    n = lambda x: None if x is None else x.detach().double().numpy()
    if T % 64:
        # the oracle works on whole chunks: pad exactly like the backend does
        pad = 64 - T % 64
        P = lambda x: None if x is None else np.concatenate([n(x), np.zeros((x.shape[0], pad) + tuple(x.shape[2:]))], 1)
        ref = O.backward(op, P(xs["q"]), P(xs["k"]), P(xs["v"]), g=P(xs.get("g")), beta=P(xs.get("beta")),
                         b=P(xs.get("b")), w=P(xs.get("w")), h0=n(xs["initial_state"]), dO=P(dO), dht=n(dht))
        ref = {k: (v[:, :T] if isinstance(v, np.ndarray) and v.ndim >= 3 and v.shape[1] == T + pad else v)
               for k, v in ref.items()}
    else:
        ref = O.backward(op, n(xs["q"]), n(xs["k"]), n(xs["v"]), g=n(xs.get("g")), beta=n(xs.get("beta")),
                         b=n(xs.get("b")), w=n(xs.get("w")), h0=n(xs["initial_state"]), dO=n(dO), dht=n(dht))
    for (name, _), gr in zip(xg.items(), grads):
        e = O.error(ref[GRAD[name]], n(gr), O.limit_for(GRAD[name]))
        assert e["passed"], (name, e)
