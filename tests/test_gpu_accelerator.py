"""The reference's accelerator cases on the HIP path (reference tests/test_accelerator.py).

* absent ``initial_state`` with a non-contiguous ``q`` for every family
  (test_accelerator.py:33-48): optimized against the original backend, and against
  the fp64 oracle, at the reference's tolerances (rel-L2 0.008, 0.02 for g/beta/b/w);
* KDA's model-gate combination (test_accelerator.py:65-83): ``use_gate_in_kernel`` +
  ``use_beta_sigmoid_in_kernel`` + ``use_qk_l2norm_in_kernel`` + ``state_v_first``, with
  gradients of every leaf (q, k, v, raw g, raw beta, A_log, dt_bias, initial_state) and the
  outputs o / final state compared between backends;
* the beta sigmoid with ``allow_neg_eigval`` (scale 2) for KDA and GDN, whose backward is
  folded into the chunk kernel's dbeta stores;
* the folded gate with ``lower_bound`` and no ``A_log``, and with a chunk-aligned
  ``cu_seqlens`` batch (no padded tokens: the fold applies there too).

Inputs follow the reference's ``validation.inputs`` distributions (validation.py:6-21:
raw per-token log gates -U(0, 0.05), beta U(0.1, 0.9) in bf16, h0 ~ N(0, 0.05^2)),
restated here; the original backend is this package's PyTorch 7-product formulation.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu

OPNAME = {"kda": "chunk_kda", "gdn": "chunk_gated_delta_rule", "gdn2": "chunk_gdn2", "delta": "chunk_delta_rule"}
LOOSE = ("g", "beta", "b", "w", "A_log", "dt_bias")


def ref_inputs(op, length=128, heads=2, seed=42, batch=1):
    """validation.py:6-21's distributions on the CPU (seeded), bf16 q/k/v/beta."""
    gen = torch.Generator().manual_seed(seed)
    shape = (batch, length, heads, 128)
    q = F.normalize(torch.randn(shape, generator=gen), dim=-1).bfloat16()
    k = F.normalize(torch.randn(shape, generator=gen), dim=-1).bfloat16()
    v = torch.randn(shape, generator=gen).bfloat16()
    xs = dict(q=q, k=k, v=v)
    if op != "delta":
        xs["g"] = -torch.rand(shape[:-1] if op == "gdn" else shape, generator=gen) * 0.05
    if op == "gdn2":
        xs["b"] = (torch.rand(shape, generator=gen) * 0.8 + 0.1).bfloat16()
        xs["w"] = (torch.rand(shape, generator=gen) * 0.8 + 0.1).bfloat16()
    else:
        xs["beta"] = (torch.rand(shape[:-1], generator=gen) * 0.8 + 0.1).bfloat16()
    xs["initial_state"] = torch.randn((batch, heads, 128, 128), generator=gen) * 0.05
    return xs


def _leaves(xs, dev):
    return {n: x.to(dev).detach().requires_grad_() for n, x in xs.items()}


def _grads(op, xs, dO, backend, dht=None, **kw):
    import rewy_amd as fdr
    with fdr.use_backend(backend, ops=(op,)):
        o, ht = getattr(fdr, OPNAME[op])(**xs, **kw)
    outs, cots = (o,), (dO,)
    if dht is not None:
        outs, cots = (o, ht), (dO, dht)
    grads = torch.autograd.grad(outs, tuple(xs.values()), cots)
    torch.cuda.synchronize()
    return o, ht, dict(zip(xs, grads))


def _compare(ref, got, names=None):
    for name in names or ref:
        lim = 0.02 if name in LOOSE else 0.008
        e = O.error(ref[name].detach().double().cpu().numpy(), got[name].detach().double().cpu().numpy(), lim)
        print(f"  {name}: rel-L2 {e['relative_l2']:.2e} max-abs {e['max_abs']:.2e}", flush=True)
        assert e["passed"], (name, e)


@pytest.mark.parametrize("op", ["kda", "gdn", "gdn2", "delta"])
def test_absent_state_and_noncontiguous_input(op):
    """test_accelerator.py:33-48: no initial_state, q strided (T and H swapped in memory)."""
    import rewy_amd as fdr
    print(f"\n[accel] absent h0 + non-contiguous q op={op}", flush=True)
    dev = torch.device("cuda")
    cpu = ref_inputs(op, length=128)
    cpu.pop("initial_state")
    xs = _leaves(cpu, dev)
    xs["q"] = xs["q"].detach().transpose(1, 2).contiguous().transpose(1, 2).requires_grad_()
    assert not xs["q"].is_contiguous()
    dO = torch.randn(xs["v"].shape, generator=torch.Generator().manual_seed(7)).bfloat16().to(dev)
    kw = dict(disable_recompute=True) if op in ("kda", "gdn2") else {}
    # the public operators take raw per-token gates; the oracle takes the same raw gates
    fdr.stats(reset=True)
    o_opt, _, g_opt = _grads(op, xs, dO, "optimized", **kw)
    fdr.assert_used((op,))
    assert not any("fallback" in k or "rejected" in k for k in fdr.stats())
    o_ref, _, g_ref = _grads(op, xs, dO, "original", **kw)
    print(" vs original backend", flush=True)
    _compare(g_ref, g_opt)
    _compare(dict(o=o_ref), dict(o=o_opt))
    n = lambda x: None if x is None else x.detach().double().cpu().numpy()
    orc = O.backward(op, n(cpu["q"]), n(cpu["k"]), n(cpu["v"]), g=n(cpu.get("g")), beta=n(cpu.get("beta")),
                     b=n(cpu.get("b")), w=n(cpu.get("w")), h0=None, dO=n(dO), dht=None)
    print(" vs fp64 oracle", flush=True)
    grad = {"q": "dq", "k": "dk", "v": "dv", "g": "dg", "beta": "dbeta", "b": "db", "w": "dw"}
    for name, gv in g_opt.items():
        e = O.error(orc[grad[name]], n(gv), O.limit_for(grad[name]))
        assert e["passed"], (name, e)


@pytest.mark.parametrize("policy", ["full", "recompute"])
def test_kda_model_gate_gradients(policy):
    """test_accelerator.py:65-83: raw gate and raw beta, gate + beta sigmoid + q/k l2norm
    in kernel, V-first states; every leaf's gradient, o and the final state."""
    print(f"\n[accel] kda model gate policy={policy}", flush=True)
    dev = torch.device("cuda")
    cpu = ref_inputs("kda", length=128)
    gen = torch.Generator().manual_seed(11)
    cpu["g"] = torch.randn(cpu["q"].shape, generator=gen)
    cpu["beta"] = torch.randn(cpu["beta"].shape, generator=gen).bfloat16()
    cpu["A_log"] = torch.full((2,), -2.0)
    cpu["dt_bias"] = torch.zeros(256)
    # raw q/k (not unit norm), so the l2norm backward matters
    cpu["q"] = (torch.randn(cpu["q"].shape, generator=gen) * 2).bfloat16()
    cpu["k"] = (torch.randn(cpu["k"].shape, generator=gen) * 2).bfloat16()
    kw = dict(use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True, use_qk_l2norm_in_kernel=True,
              state_v_first=True, output_final_state=True, disable_recompute=policy == "full")
    dO = torch.randn(cpu["v"].shape, generator=gen).bfloat16().to(dev)
    dht = (torch.randn(cpu["initial_state"].shape, generator=gen) * 0.1).to(dev)
    res = {}
    for backend in ("original", "optimized"):
        xs = _leaves(cpu, dev)
        res[backend] = _grads("kda", xs, dO, backend, dht=dht, **kw)
    (o_r, h_r, g_r), (o_o, h_o, g_o) = res["original"], res["optimized"]
    _compare(dict(g_r, o=o_r, final=h_r), dict(g_o, o=o_o, final=h_o))
    assert g_o["beta"].dtype == torch.bfloat16 and g_o["A_log"].shape == (2,)


@pytest.mark.parametrize("op", ["kda", "gdn"])
@pytest.mark.parametrize("neg", [False, True])
def test_beta_sigmoid_folded_backward(op, neg):
    """use_beta_sigmoid_in_kernel (allow_neg_eigval: beta = 2 sigmoid(x)): the optimized
    backward writes dL/dx from the chunk kernel; the original backend differentiates
    torch's sigmoid.  T = 192: the fold applies (no padded tokens)."""
    import rewy_amd as fdr
    print(f"\n[accel] beta sigmoid op={op} neg={neg}", flush=True)
    dev = torch.device("cuda")
    cpu = ref_inputs(op, length=192, heads=3, seed=5)
    gen = torch.Generator().manual_seed(12)
    cpu["beta"] = torch.randn(cpu["beta"].shape, generator=gen) * 2
    cpu["beta"][:, ::9] = -30.0        # sigmoid ~ 1e-13: rows on the |beta| < 1e-6 branch
    kw = dict(use_beta_sigmoid_in_kernel=True, allow_neg_eigval=neg)
    if op == "kda":
        kw["disable_recompute"] = True
    dO = torch.randn(cpu["v"].shape, generator=gen).bfloat16().to(dev)
    dht = (torch.randn(cpu["initial_state"].shape, generator=gen) * 0.1).to(dev)
    res = {}
    for backend in ("original", "optimized"):
        res[backend] = _grads(op, _leaves(cpu, dev), dO, backend, dht=dht, output_final_state=True, **kw)
    (o_r, h_r, g_r), (o_o, h_o, g_o) = res["original"], res["optimized"]
    _compare(dict(g_r, o=o_r, final=h_r), dict(g_o, o=o_o, final=h_o))
    fdr.stats(reset=True)


@pytest.mark.parametrize("case", ["lower_bound_only", "aligned_varlen"])
def test_kda_fused_gate_forms(case):
    """The folded gate backward with lower_bound = -5 and A_log = None (activation
    lower_bound * sigmoid(g + dt_bias)), and with a chunk-aligned packed batch (sequences of
    128 and 64 tokens: no padded token, so the fold applies); o, the final state and every
    leaf's gradient against the original backend."""
    print(f"\n[accel] kda fused gate {case}", flush=True)
    dev = torch.device("cuda")
    gen = torch.Generator().manual_seed(13)
    T = 192
    cpu = ref_inputs("kda", length=T, heads=2, seed=9)
    cpu["g"] = torch.randn(cpu["q"].shape, generator=gen)
    cpu["dt_bias"] = torch.randn(256, generator=gen) * 0.1
    kw = dict(use_gate_in_kernel=True, output_final_state=True, disable_recompute=True)
    if case == "lower_bound_only":
        kw["lower_bound"] = -5.0
    else:
        cpu["A_log"] = torch.randn(2, generator=gen) * 0.5
        cpu["initial_state"] = torch.cat([cpu["initial_state"]] * 2, 0)
        kw["cu_seqlens"] = torch.tensor([0, 128, T], device=dev)
    dO = torch.randn(cpu["v"].shape, generator=gen).bfloat16().to(dev)
    dht = (torch.randn(cpu["initial_state"].shape, generator=gen) * 0.1).to(dev)
    res = {}
    for backend in ("original", "optimized"):
        res[backend] = _grads("kda", _leaves(cpu, dev), dO, backend, dht=dht, **kw)
    (o_r, h_r, g_r), (o_o, h_o, g_o) = res["original"], res["optimized"]
    _compare(dict(g_r, o=o_r, final=h_r), dict(g_o, o=o_o, final=h_o))
