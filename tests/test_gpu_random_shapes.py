"""The public backward at seeded random shapes against the fp64 oracle, two heads each.

Every backend choice (affine-step, paired in one launch at 16 / 32 / 64-wide tiles, the
scan beside the segmented recurrence, the fused sweep, plain direct) is a function of
batch x heads and chunk count, so a spread of shapes walks across all of them: batch
1-3, 1-33 value heads with grouped q / k heads (G = 1, 2, 4), 1-33 chunks, both KDA / GDN2
policies, V-first states, with and without an initial state.  For each case the first and
the last (batch row, head) pairs are run through the oracle alone and compared at the
reference's tolerances (validation.py:40-45, :68).  dq / dk of grouped heads are sums over
the group (held to the oracle in test_gpu_gva.py) and are skipped here."""
import random

import pytest
import torch

from oracle import delta_oracle as O
from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu

OPNAME = {"kda": "chunk_kda", "gdn": "chunk_gated_delta_rule", "gdn2": "chunk_gdn2", "delta": "chunk_delta_rule"}
GRAD = {"q": "dq", "k": "dk", "v": "dv", "g": "dg", "beta": "dbeta", "b": "db", "w": "dw", "initial_state": "dh0"}


def _case(i):
    rng = random.Random(9000 + i)
    op = rng.choice(["kda", "gdn", "gdn2", "delta"])
    B = rng.choice([1, 1, 2, 3])
    H = rng.choice([1, 2, 3, 4, 5, 8, 12, 16, 20, 24, 33])
    T = 64 * rng.choice([1, 2, 3, 4, 5, 8, 9, 12, 16, 17, 24, 33])
    full = op in ("kda", "gdn2") and rng.random() < 0.4
    vf = op != "delta" and rng.random() < 0.3      # (the reference's DeltaNet op has no state_v_first)
    G = rng.choice([1, 1, 2, 4]) if op != "gdn2" else 1
    if H % G:
        G = 1
    h0 = op != "gdn2" or rng.random() < 0.5
    return op, B, T, H, G, full, vf, h0, rng.randrange(10 ** 6)


@pytest.mark.parametrize("i", range(48))
def test_random_shape_matches_oracle(i):
    import rewy_amd as fdr
    op, B, T, H, G, full, vf, h0, seed = _case(i)
    print(f"\n[random] op={op} B={B} T={T} H={H} G={G} full_saving={full} state_v_first={vf} h0={h0}", flush=True)
    dev = torch.device("cuda")
    xs, dO = make_inputs(op, B, T, H, seed=seed, gate="mild" if op in ("kda", "gdn2") else "default", h0=h0)
    if G > 1:
        xs["q"], xs["k"] = xs["q"][:, :, ::G].contiguous(), xs["k"][:, :, ::G].contiguous()
    leaves = {n: v.to(dev).requires_grad_() for n, v in xs.items() if v is not None}
    if vf and "initial_state" in leaves:
        leaves["initial_state"] = xs["initial_state"].transpose(-1, -2).contiguous().to(dev).requires_grad_()
    kw = dict(disable_recompute=full) if op in ("kda", "gdn2") else {}
    if vf:
        kw["state_v_first"] = True
    with fdr.use_backend("optimized", ops=(op,)):
        o, ht = getattr(fdr, OPNAME[op])(**leaves, output_final_state=True, **kw)
    dht = torch.randn(ht.shape, generator=torch.Generator().manual_seed(7)) * 0.05
    grads = dict(zip(leaves, torch.autograd.grad((o, ht), list(leaves.values()), (dO.to(dev), dht.to(dev)))))
    torch.cuda.synchronize()
    fdr.assert_used((op,))
    for bb, hh in ((0, 0), (B - 1, H - 1)):
        def head(x, name, transposed=False):
            x = x.detach()
            if name in ("initial_state", "dht"):
                x = x[bb:bb + 1, hh:hh + 1]
                if transposed:
                    x = x.transpose(-1, -2)
            else:
                j = hh // G if name in ("q", "k") else hh
                x = x[bb:bb + 1, :, j:j + 1]
            return x.double().cpu().numpy()
        opt = lambda n: head(xs[n], n) if xs.get(n) is not None else None
        ref = O.backward(op, head(xs["q"], "q"), head(xs["k"], "k"), head(xs["v"], "v"), g=opt("g"),
                         beta=opt("beta"), b=opt("b"), w=opt("w"), h0=opt("initial_state"), dO=head(dO, "dO"),
                         dht=head(dht, "dht", vf))
        report = {}
        for name, gr in grads.items():
            if G > 1 and name in ("q", "k"):
                continue
            e = O.error(ref[GRAD[name]], head(gr, name, vf and name == "initial_state"), O.limit_for(GRAD[name]))
            report[name] = round(e["relative_l2"], 5)
            assert e["passed"], (op, B, T, H, G, full, vf, (bb, hh), name, e)
        print(f"head ({bb}, {hh}) rel-L2 vs fp64 oracle", report, flush=True)
