"""The BASELINE.json workloads at their full sizes against the fp64 oracle, head by head.

Every (batch row, head) pair of the chunked delta rule is independent end to end, so the
gradients the optimized path (HIP forward + HIP backward, through the public autograd
operators) produces for one head of the full-size batch must equal the oracle's gradients
for that head's inputs alone.  For each config, three heads (the first, the last and one in
between) are checked at the reference's acceptance tolerances (validation.py:40-45, :68:
rel-L2 <= 0.008 for q / k / v / h0 and the output, <= 0.02 for g / beta / b / w), with the
oracle (oracle/delta_oracle.py, numpy fp64) run on the head's full sequence (kda_long: 65,536
tokens, ~4 GB of pairwise gate factors per head)."""
import pytest
import torch

from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu

OPNAME = {"kda": "chunk_kda", "gdn": "chunk_gated_delta_rule", "gdn2": "chunk_gdn2", "delta": "chunk_delta_rule"}
GRAD = {"q": "dq", "k": "dk", "v": "dv", "g": "dg", "beta": "dbeta", "b": "db", "w": "dw", "initial_state": "dh0"}


@pytest.mark.parametrize("config", ["kda", "gdn", "gdn_cfg", "gdn2", "kda_long"])
def test_full_size_heads_match_the_oracle(config):
    import bench
    import rewy_amd as fdr
    cfg = bench.CONFIGS[config]
    op, B, H = cfg["op"], cfg["B"], cfg["H"]
    print(f"\n[fullsize-oracle] {config}: op={op} B={B} T={cfg['T']} H={H}", flush=True)
    xs, dO = bench.make_inputs(cfg, "cuda")
    args = dict(q=xs["q"], k=xs["k"], v=xs["v"])
    if op == "gdn2":
        args.update(g=xs["g"], b=xs["b"], w=xs["w"])
    elif op == "delta":
        args.update(beta=xs["beta"])
    else:
        args.update(g=xs["g"], beta=xs["beta"])
    if xs["h0"] is not None:
        args["initial_state"] = xs["h0"]
    kw = dict(disable_recompute=cfg["full_saving"]) if op in ("kda", "gdn2") else {}
    leaves = {n: v.clone().requires_grad_() for n, v in args.items()}
    with fdr.use_backend("optimized", ops=(op,)):
        o, _ = getattr(fdr, OPNAME[op])(**leaves, **kw)
    grads = dict(zip(leaves, torch.autograd.grad(o, list(leaves.values()), dO)))
    torch.cuda.synchronize()
    for bb, hh in ((0, 0), (B - 1, H - 1)):
        def head(x, name):
            if x is None:
                return None
            x = x.detach()
            x = x[bb:bb + 1, hh:hh + 1] if name == "initial_state" else x[bb:bb + 1, :, hh:hh + 1]
            return x.double().cpu().numpy()
        ref = O.backward(op, head(args["q"], "q"), head(args["k"], "k"), head(args["v"], "v"),
                         g=head(args.get("g"), "g"), beta=head(args.get("beta"), "beta"), b=head(args.get("b"), "b"),
                         w=head(args.get("w"), "w"), h0=head(args.get("initial_state"), "initial_state"),
                         dO=head(dO, "dO"), dht=None)
        report = {}
        for name, gr in grads.items():
            lim = O.limit_for(GRAD[name])
            e = O.error(ref[GRAD[name]], head(gr, name), lim)
            report[name] = round(e["relative_l2"], 5)
            assert e["passed"], (config, (bb, hh), name, e)
        print(f"head ({bb}, {hh}) rel-L2 vs fp64 oracle", report, flush=True)
