"""End-to-end gradients of the public operators on the GPU.

The optimized (HIP) backward is compared with the fp64 oracle (token-recurrence
pinned) at the reference's acceptance tolerances (validation.py:40-45 and
:68: rel-L2 <= 0.008 for q/k/v/h0, <= 0.02 for g/beta/b/w) and with the
original-formulation backend on the same inputs (test_accelerator.py:7-31).
"""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu

OPNAME = {"kda": "chunk_kda", "gdn": "chunk_gated_delta_rule", "gdn2": "chunk_gdn2", "delta": "chunk_delta_rule"}
GRAD = {"q": "dq", "k": "dk", "v": "dv", "g": "dg", "beta": "dbeta", "b": "db", "w": "dw", "initial_state": "dh0"}


def _run(op, xs, dO, backend, **kw):
    import rewy_amd as fdr
    dev = torch.device("cuda")
    xg = {k: v.to(dev).requires_grad_() for k, v in xs.items()}
    with fdr.use_backend(backend, ops=(op,)):
        o, ht = getattr(fdr, OPNAME[op])(**xg, output_final_state=True, **kw)
    dht = (torch.randn(ht.shape, generator=torch.Generator().manual_seed(9)) * 0.1).to(dev)
    grads = torch.autograd.grad((o, ht), tuple(xg.values()), (dO.to(dev), dht))
    torch.cuda.synchronize()
    return dict(zip(xs, grads)), dht.cpu()


@pytest.mark.parametrize("op,kw", [("kda", dict(disable_recompute=True)), ("kda", dict(disable_recompute=False)),
                                   ("gdn", {}), ("gdn2", dict(disable_recompute=True)), ("delta", {})])
# T = 640: ten chunks at B*H = 4, so the recompute policy's forward and backward state
# recurrences take the affine-step kernels (at most 8 chunks take the paired direct recurrences,
# in one launch; the full-saving policy's state recurrence alone is direct up to 16 chunks)
@pytest.mark.parametrize("T", [128, 320, 640])
def test_public_backward_matches_oracle(op, kw, T):
    import rewy_amd as fdr
    print(f"\n[e2e] op={op} kw={kw} T={T}", flush=True)
    xs, dO = make_inputs(op, 2, T, 2, seed=21, beta_zero_every=7 if op != "gdn2" else 0)
    fdr.stats(reset=True)
    got, dht = _run(op, xs, dO, "optimized", **kw)
    fdr.assert_used((op,))
    assert not any("fallback" in k or "rejected" in k for k in fdr.stats())
    n = lambda x: None if x is None else x.detach().double().cpu().numpy()
    ref = O.backward(op, n(xs["q"]), n(xs["k"]), n(xs["v"]), g=n(xs.get("g")), beta=n(xs.get("beta")),
                     b=n(xs.get("b")), w=n(xs.get("w")), h0=n(xs["initial_state"]), dO=n(dO), dht=n(dht))
    report = {}
    for name, grad in got.items():
        e = O.error(ref[GRAD[name]], n(grad), O.limit_for(GRAD[name]))
        report[name] = (round(e["relative_l2"], 5), e["max_abs"])
        assert e["passed"], (name, e)
    print("rel-L2/max-abs vs oracle", report, flush=True)


@pytest.mark.parametrize("op", ["kda", "gdn", "gdn2", "delta"])
def test_optimized_matches_original_backend(op):
    print(f"\n[e2e-orig] op={op}", flush=True)
    xs, dO = make_inputs(op, 1, 256, 3, seed=33)
    kw = dict(disable_recompute=True) if op in ("kda", "gdn2") else {}
    a, _ = _run(op, xs, dO, "optimized", **kw)
    b, _ = _run(op, xs, dO, "original", **kw)
    for name in a:
        e = O.error(b[name].double().cpu().numpy(), a[name].double().cpu().numpy(), O.limit_for(GRAD[name]))
        assert e["passed"], (name, e)


@pytest.mark.parametrize("op", ["kda", "gdn", "gdn2", "delta"])
def test_optimized_matches_original_with_l2norm_in_kernel(op):
    """use_qk_l2norm_in_kernel: the optimized backend normalises q / k with the HIP
    kernels, the original backend with torch ops; raw (unnormalised) q / k in."""
    print(f"\n[e2e-l2norm] op={op}", flush=True)
    xs, dO = make_inputs(op, 1, 192, 2, seed=35)
    gen = torch.Generator().manual_seed(36)
    xs["q"] = (torch.randn(xs["q"].shape, generator=gen) * 3).bfloat16()
    xs["k"] = (torch.randn(xs["k"].shape, generator=gen) * 3).bfloat16()
    kw = dict(use_qk_l2norm_in_kernel=True)
    if op in ("kda", "gdn2"):
        kw["disable_recompute"] = True
    a, _ = _run(op, xs, dO, "optimized", **kw)
    b, _ = _run(op, xs, dO, "original", **kw)
    for name in a:
        e = O.error(b[name].double().cpu().numpy(), a[name].double().cpu().numpy(), O.limit_for(GRAD[name]))
        assert e["passed"], (name, e)


def test_backward_stays_bound_after_disable():
    import rewy_amd as fdr
    xs, dO = make_inputs("kda", 1, 128, 2, seed=3)
    dev = torch.device("cuda")
    xg = {k: v.to(dev).requires_grad_() for k, v in xs.items()}
    fdr.stats(reset=True)
    fdr.enable("optimized", ops=("kda",))
    o, _ = fdr.chunk_kda(**xg)
    fdr.disable()
    torch.autograd.grad(o, tuple(xg.values()), dO.to(dev))
    fdr.assert_used(("kda",))


def test_rejection_and_visible_fallback():
    import rewy_amd as fdr
    xs, dO = make_inputs("kda", 1, 128, 2, seed=3)
    dev = torch.device("cuda")
    xg = {k: v[:, :65].contiguous().to(dev).requires_grad_() if v.ndim > 3 or k == "beta" else v.to(dev).requires_grad_()
          for k, v in xs.items()}
    with fdr.use_backend("optimized"):
        with pytest.raises(RuntimeError, match="multiple of 64"):
            fdr.chunk_kda(**xg)
    fdr.stats(reset=True)
    with fdr.use_backend("optimized", strict=False):
        with pytest.warns(RuntimeWarning, match="using original"):
            out, _ = fdr.chunk_kda(**xg)
    out.float().sum().backward()
    assert fdr.stats()["kda.fallback_forward"] == 1
    assert fdr.stats().get("kda.optimized_backward", 0) == 0


@pytest.mark.parametrize("lower_bound,with_a_log", [(None, True), (-5.0, True), (-5.0, False)])
# the activation and its backward run inside the chunk Function (folded into the chunk
# kernel): T = 128 dense rows; T = 192 as one packed row with a ragged cu_seqlens (partial
# chunks, fdr_chunk_bwd_gate_fold_varlen)
@pytest.mark.parametrize("T", [128, 192])
def test_kda_fused_gate_optimized_matches_original(lower_bound, with_a_log, T):
    """use_gate_in_kernel=True (the gate activation feeding the HIP backward, dA_log /
    ddt_bias through its explicit backward) against the original backend on the
    same inputs: the output and every leaf's gradient (q, k, v, beta, g_raw, A_log, dt_bias);
    the lower-bound form with and without A_log; and the envelope: accepted for KDA,
    rejected for GDN / GDN2 with the reference's reasons (runtime.py:97-98)."""
    import rewy_amd as fdr
    from rewy_amd.runtime import rejection_reason
    print(f"\n[e2e] kda fused gate lower_bound={lower_bound} A_log={with_a_log} T={T}", flush=True)
    xs, dO = make_inputs("kda", 2, T, 2, seed=31)
    gen = torch.Generator().manual_seed(5)
    leaves = dict(q=xs["q"], k=xs["k"], v=xs["v"], beta=xs["beta"], g=torch.randn(2, T, 2, 128, generator=gen),
                  A_log=torch.randn(2, generator=gen) * 0.5, dt_bias=torch.randn(256, generator=gen) * 0.1)
    if not with_a_log:
        del leaves["A_log"]
    dev = torch.device("cuda")
    res = {}
    for backend in ("optimized", "original"):
        lv = {k: v.to(dev).requires_grad_() for k, v in leaves.items()}
        with fdr.use_backend(backend, ops=("kda",)):
            packed = dict(cu_seqlens=torch.tensor([0, 70, T], device=dev)) if T == 192 else {}
            if packed:     # one packed row of two sequences, one initial state each
                flat = lambda x: x.reshape(1, 2 * T, *x.shape[2:])
                args = [flat(lv["q"]), flat(lv["k"]), flat(lv["v"]), flat(lv["g"]), flat(lv["beta"])]
                packed["cu_seqlens"] = torch.tensor([0, 70, 2 * T], device=dev)
            else:
                args = [lv["q"], lv["k"], lv["v"], lv["g"], lv["beta"]]
            o, _ = fdr.chunk_kda(*args, initial_state=xs["initial_state"].to(dev), use_gate_in_kernel=True,
                                 A_log=lv.get("A_log"), dt_bias=lv["dt_bias"], lower_bound=lower_bound, **packed)
        grads = torch.autograd.grad(o, list(lv.values()), dO.to(dev).reshape(o.shape))
        res[backend] = [o.detach().double().cpu().numpy()] + [x.detach().double().cpu().numpy() for x in grads]
    for name, a, r in zip(["o"] + list(leaves), res["optimized"], res["original"]):
        e = O.error(r, a, 0.02 if name in ("g", "A_log", "dt_bias", "beta") else 0.008)
        print(name, e, flush=True)
        assert e["passed"], (name, e)
    q = xs["q"].to(dev)
    assert rejection_reason("kda", dict(q=q, k=q, v=q, use_gate_in_kernel=True)) is None
    assert rejection_reason("gdn", dict(q=q, k=q, v=q, use_gate_in_kernel=True)) == "GDN fused gate is not release-validated"
    assert rejection_reason("gdn2", dict(q=q, k=q, v=q, use_gate_in_kernel=True)) == "GDN2 fused gate is not release-validated"


@pytest.mark.parametrize("op", ["kda", "gdn", "gdn2", "delta"])
def test_optimized_varlen_and_v_first_match_original(op):
    """Packed sequences (cu_seqlens, lengths not multiples of 64) and V-first states
    on the HIP path against the original backend on the same inputs; grouped value
    heads stay outside GDN2's optimized envelope (the reference's reason)."""
    import rewy_amd as fdr
    print(f"\n[e2e] varlen / state_v_first op={op}", flush=True)
    lens = [100, 128, 37]
    dev = torch.device("cuda")
    seqs = [make_inputs(op, 1, L, 2, seed=70 + i) for i, L in enumerate(lens)]
    names = [n for n in seqs[0][0] if n != "initial_state"]
    packed = {n: torch.cat([x[n] for x, _ in seqs], 1).to(dev) for n in names}
    packed["initial_state"] = torch.cat([x["initial_state"] for x, _ in seqs], 0).transpose(-1, -2).contiguous().to(dev)
    dO = torch.cat([d for _, d in seqs], 1).to(dev)
    cu = torch.tensor([0, 100, 228, 265], device=dev)
    kw = dict(cu_seqlens=cu, output_final_state=True)
    if op != "delta":
        kw["state_v_first"] = True
    else:
        packed["initial_state"] = packed["initial_state"].transpose(-1, -2).contiguous()
    if op in ("kda", "gdn2"):
        kw["disable_recompute"] = True
    res = {}
    for backend in ("optimized", "original"):
        fdr.stats(reset=True)
        xg = {n: v.clone().requires_grad_() for n, v in packed.items()}
        with fdr.use_backend(backend, ops=(op,)):
            o, ht = getattr(fdr, OPNAME[op])(**xg, **kw)
        dht = (torch.randn(ht.shape, generator=torch.Generator().manual_seed(4)) * 0.1).to(dev)
        res[backend] = [o] + list(torch.autograd.grad((o, ht), list(xg.values()), (dO, dht))) + [ht]
        if backend == "optimized":
            fdr.assert_used((op,))
    for name, a, r in zip(["o"] + list(packed) + ["final"], res["optimized"], res["original"]):
        lim = 0.02 if name in ("g", "beta", "b", "w") else 0.008
        e = O.error(r.detach().double().cpu().numpy(), a.detach().double().cpu().numpy(), lim)
        print(name, e, flush=True)
        assert e["passed"], (name, e)
    if op == "gdn2":
        # grouped value heads run natively for KDA, GDN and DeltaNet (tests/test_gpu_gva.py);
        # GDN2's operator defines none, so the envelope keeps the reference's rejection
        xs, _ = make_inputs(op, 1, 128, 4, seed=3)
        q2 = xs["q"][:, :, ::2].contiguous().to(dev)
        args = {n: v.to(dev) for n, v in xs.items()}
        args.update(q=q2, k=q2)
        with fdr.use_backend("optimized", ops=(op,)):
            with pytest.raises(RuntimeError, match="grouped heads or unequal q/k/v shapes"):
                getattr(fdr, OPNAME[op])(**args)
