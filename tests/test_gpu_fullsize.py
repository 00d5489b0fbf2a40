"""The BASELINE.json workloads at their full sizes: the optimized path (HIP
forward + HIP backward) against the original-formulation backend (PyTorch ops,
fp32) on the same inputs, through the public autograd operators, at the
reference's acceptance tolerances (validation.py:40-45: rel-L2 <= 0.008 for
q/k/v/h0 gradients and the output, <= 0.02 for g/beta/b/w)."""
import pytest
import torch

from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu

OPNAME = {"kda": "chunk_kda", "gdn": "chunk_gated_delta_rule", "gdn2": "chunk_gdn2", "delta": "chunk_delta_rule"}


@pytest.mark.parametrize("config", ["kda", "gdn", "gdn_cfg", "gdn2", "kda_long"])
def test_full_size_optimized_matches_original(config):
    import bench
    import rewy_amd as fdr
    cfg = bench.CONFIGS[config]
    op = cfg["op"]
    print(f"\n[fullsize] {config}: op={op} B={cfg['B']} T={cfg['T']} H={cfg['H']}", flush=True)
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
    res = {}
    for backend in ("optimized", "original"):
        leaves = {n: v.clone().requires_grad_() for n, v in args.items()}
        with fdr.use_backend(backend, ops=(op,)):
            o, _ = getattr(fdr, OPNAME[op])(**leaves, **kw)
        grads = torch.autograd.grad(o, list(leaves.values()), dO)
        res[backend] = [o.detach()] + [g.detach() for g in grads]
        del o, grads, leaves
        torch.cuda.synchronize()
    for name, a, r in zip(["o"] + list(args), res["optimized"], res["original"]):
        lim = 0.02 if name in ("g", "beta", "b", "w") else 0.008
        e = O.error(r.double().cpu().numpy(), a.double().cpu().numpy(), lim)
        print(name, {k: (round(v, 6) if isinstance(v, float) else v) for k, v in e.items()}, flush=True)
        assert e["passed"], (config, name, e)
