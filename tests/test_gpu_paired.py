"""The recompute policy's paired direct recurrences (17 <= B*H <= 127, and B*H <= 16 on short
rows): the direct backward state recurrence and the direct forward scan side by side in one
launch (fdr_paired_recurrences), at the value-tile width ``ops.paired_tile`` picks (32 at
B*H = 32, 64 at B*H = 48, 16 at B*H = 16 with few chunks).  For all four families (the
scalar / no-gate ones with the state recurrence forming Aqk itself):

* the public autograd backward (recompute policy) against the fp64 oracle at the
  reference's acceptance tolerances (validation.py:40-45, :68);
* the same gradients, bit for bit, whether GDN / DeltaNet's three launches are made by one
  library call (fdr_scalar_bwd, ``ops.SCALAR_ONE_CALL``) or one by one, whether the two
  recurrences run as one launch
  (fdr_paired_recurrences, ``ops.PAIRED_ONE_LAUNCH``) or as two launches on two streams, as
  the same launches enqueued on one stream, as the two
  recurrences reading the w (``ops.PAIRED_FORMW`` off, GDN2) and the qg / kg (``ops.PAIRED_RAW``
  off) that prepare_wu wrote instead of forming them from the raw q / k, and as the scan reading a u that prepare_wu wrote
  (``ops.PAIRED_U`` off: the scan forms u itself);
* against the policy switched off (the pair one after the other at the default tile
  width): rel-L2 <= 1e-5, the tile width changing no arithmetic of a value column (5e-3 for the
  scalar / no-gate families at narrow tiles, where the pair reads the Aqk fdr_prepare_wu writes
  instead of forming it);
* captured in a HIP graph and replayed three times with eager work between the replays.
"""
import pytest
import torch

from oracle import delta_oracle as O
from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu

OPNAME = {"kda": "chunk_kda", "gdn2": "chunk_gdn2", "gdn": "chunk_gated_delta_rule", "delta": "chunk_delta_rule"}
OPS = ["kda", "gdn2", "gdn", "delta"]
GATE = {"kda": 2, "gdn2": 2, "gdn": 1, "delta": 0}
GRAD = {"q": "dq", "k": "dk", "v": "dv", "g": "dg", "beta": "dbeta", "b": "db", "w": "dw", "initial_state": "dh0"}
SHAPES = [(2, 512, 16, 32), (1, 256, 48, 64), (1, 512, 16, 16)]    # B, T, H, the tile width paired_tile picks


def _count_pairs(monkeypatch):
    """Count the paired recurrences: one launch (ops.paired_recurrences, or inside the one-call
    GDN / DeltaNet backward ops.scalar_bwd) or two streams."""
    from rewy_amd import ops
    from rewy_amd.backends import backward as bw
    calls = []
    real_sbs, real_one, real_scalar = bw._side_by_side, ops.paired_recurrences, ops.scalar_bwd
    monkeypatch.setattr(bw, "_side_by_side", lambda a, b: (calls.append("streams"), real_sbs(a, b))[1])
    monkeypatch.setattr(ops, "paired_recurrences", lambda *a, **k: (calls.append("one"), real_one(*a, **k))[1])
    monkeypatch.setattr(ops, "scalar_bwd", lambda *a, **k: (calls.append("one"), real_scalar(*a, **k))[1])
    return calls


def _rel(a, r):
    a, r = a.double(), r.double()
    return float((a - r).norm() / r.norm().clamp_min(1e-30))


def _seam(op, B, T, H):
    """The backward seam of `op` (recompute policy) on fixed inputs, as a closure."""
    from rewy_amd.backends import backward as bw
    from rewy_amd.hip_forward import chunk_forward_hip
    dev = torch.device("cuda")
    xs, dO = make_inputs(op, B, T, H, seed=51, gate="mild" if op in ("kda", "gdn2") else "default")
    xs = {n: (None if v is None else v.to(dev)) for n, v in xs.items()}
    dO = dO.to(dev)
    _, _, sv = chunk_forward_hip(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"),
                                 b=xs.get("b"), w=xs.get("w"), initial_state=xs["initial_state"])
    dht = torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(5)).mul(0.1).to(dev)
    common = dict(q=xs["q"], k=xs["k"], v=xs["v"], scale=sv["scale"], initial_state=xs["initial_state"], do=dO,
                  dht=dht)
    if op == "kda":
        return lambda: bw.kda_backward(beta=xs["beta"], Aqk=sv["Aqk"], Akk=sv["Akk"], g=sv["gc"], **common)[:6]
    if op == "gdn2":
        return lambda: bw.gdn2_backward(b=xs["b"], w_gate=xs["w"], Aqk=sv["Aqk"], Akk=sv["Akk"], g=sv["gc"],
                                        **common)[:7]
    if op == "gdn":
        return lambda: bw.gdn_backward(g=sv["gc"], beta=xs["beta"], A=sv["Akk"], **common)[:6]
    return lambda: bw.delta_backward(beta=xs["beta"], A=sv["Akk"], **common)


@pytest.mark.parametrize("B,T,H,vb", SHAPES)
@pytest.mark.parametrize("op", OPS)
def test_paired_public_backward_matches_oracle(op, B, T, H, vb, monkeypatch):
    import rewy_amd as fdr
    from rewy_amd import ops
    from rewy_amd.backends import backward as bw
    print(f"\n[paired] op={op} B={B} T={T} H={H}", flush=True)
    assert ops.paired_tile(B, H, T // 64, GATE[op]) == vb
    calls = _count_pairs(monkeypatch)
    xs, dO = make_inputs(op, B, T, H, seed=52, gate="mild" if op in ("kda", "gdn2") else "default")
    dev = torch.device("cuda")
    xg = {k: v.to(dev).requires_grad_() for k, v in xs.items()}
    kw = dict(disable_recompute=False) if op in ("kda", "gdn2") else {}
    with fdr.use_backend("optimized", ops=(op,)):
        o, ht = getattr(fdr, OPNAME[op])(**xg, output_final_state=True, **kw)
    dht = (torch.randn(ht.shape, generator=torch.Generator().manual_seed(9)) * 0.1).to(dev)
    grads = torch.autograd.grad((o, ht), tuple(xg.values()), (dO.to(dev), dht))
    torch.cuda.synchronize()
    assert calls == ["one"], calls
    n = lambda x: None if x is None else x.detach().double().cpu().numpy()
    ref = O.backward(op, n(xs["q"]), n(xs["k"]), n(xs["v"]), g=n(xs.get("g")), beta=n(xs.get("beta")),
                     b=n(xs.get("b")), w=n(xs.get("w")), h0=n(xs["initial_state"]), dO=n(dO), dht=n(dht))
    report = {}
    for name, grad in zip(xs, grads):
        e = O.error(ref[GRAD[name]], n(grad), O.limit_for(GRAD[name]))
        report[name] = round(e["relative_l2"], 5)
        assert e["passed"], (name, e)
    print("rel-L2 vs oracle", report, flush=True)


@pytest.mark.parametrize("B,T,H,vb", SHAPES)
@pytest.mark.parametrize("op", OPS)
def test_paired_equals_one_stream_and_policy_off(op, B, T, H, vb, monkeypatch):
    from rewy_amd import ops
    from rewy_amd.backends import backward as bw
    print(f"\n[paired-streams] op={op} B={B} T={T} H={H}", flush=True)
    run = _seam(op, B, T, H)
    got = [x.clone() for x in run()]
    # GDN / DeltaNet: the one-call backward (fdr_scalar_bwd) against its three launches made
    # one by one (fdr_prepare_wu, fdr_paired_recurrences, fdr_chunk_bwd)
    monkeypatch.setattr(ops, "SCALAR_ONE_CALL", False)
    three = run()
    torch.cuda.synchronize()
    for i, (a, r) in enumerate(zip(got, three)):
        assert torch.equal(a, r), (op, "SCALAR_ONE_CALL", i)
    # the two recurrences as two launches on two streams (fdr_state_bwd*, fdr_fwd_h_u)
    monkeypatch.setattr(ops, "PAIRED_ONE_LAUNCH", False)
    two = run()
    torch.cuda.synchronize()
    for i, (a, r) in enumerate(zip(got, two)):
        assert torch.equal(a, r), (op, "two launches", i)
    monkeypatch.setattr(bw, "_side_by_side", lambda first, second: (first(), second()))
    one = run()
    torch.cuda.synchronize()
    for i, (a, r) in enumerate(zip(got, one)):
        assert torch.equal(a, r), (op, i)
    monkeypatch.undo()
    # vector gates: qg / kg written by prepare_wu and read back instead of formed in the two
    # recurrences: the same bits
    monkeypatch.setattr(ops, "PAIRED_FORMW", False)
    prepared = run()
    torch.cuda.synchronize()
    for i, (a, r) in enumerate(zip(got, prepared)):
        assert torch.equal(a, r), (op, "PAIRED_FORMW", i)
    monkeypatch.setattr(ops, "PAIRED_RAW", False)
    written = run()
    torch.cuda.synchronize()
    for i, (a, r) in enumerate(zip(got, written)):
        assert torch.equal(a, r), (op, "PAIRED_RAW", i)
    monkeypatch.undo()
    # u written by prepare_wu and read by fdr_fwd_h instead of formed in the scan: the same bits
    monkeypatch.setattr(ops, "PAIRED_U", False)
    unfolded = run()
    torch.cuda.synchronize()
    for i, (a, r) in enumerate(zip(got, unfolded)):
        assert torch.equal(a, r), (op, "PAIRED_U", i)
    monkeypatch.setattr(ops, "PAIRED", False)
    # (B*H = 16 would take the affine-step form, whose rounding differs: the direct kernels)
    monkeypatch.setattr(ops, "AFFINE_MAX_BH", -1)
    off = run()
    torch.cuda.synchronize()
    # (scalar / no gate at tiles up to ops.PAIRED_AQK_MAX_VB: the pair's state recurrence reads
    # the Aqk fdr_prepare_wu writes, the unpaired one forms Aqk itself -- two bf16 roundings of
    # the same scores; both are held to the oracle in test_paired_public_backward_matches_oracle)
    tol = 5e-3 if GATE[op] != 2 and vb <= ops.PAIRED_AQK_MAX_VB else 1e-5
    for i, (a, r) in enumerate(zip(got, off)):
        e = _rel(a, r)
        assert e <= tol, (op, i, e)


@pytest.mark.parametrize("op", ["kda", "gdn"])
def test_paired_under_graph_capture(op):
    B, T, H, _ = SHAPES[0]
    print(f"\n[paired-graph] op={op} B={B} T={T} H={H}", flush=True)
    run = _seam(op, B, T, H)
    eager = [x.clone() for x in run()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        held = run()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, r) in enumerate(zip(held, eager)):
            assert torch.equal(a, r), (op, rep, i)
        run()          # eager work between the replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("op,HV,HQ", [("kda", 48, 12), ("kda", 32, 8), ("gdn", 48, 12), ("gdn2", 48, 48),
                                       ("kda", 16, 4), ("delta", 8, 2)])
def test_paired_grouped_heads_and_absent_states(op, HV, HQ, monkeypatch):
    """Grouped value heads (q / k with HQ heads) through the paired recurrences -- the raw q / k
    forms at 64-wide tiles, prepare_wu's qg / kg at 32-wide ones -- and GDN2's prepare-free form
    with no initial state and no final-state gradient: the public backward against the
    policy switched off (the recurrences one after the other), rel-L2 <= 1e-5."""
    import rewy_amd as fdr
    from rewy_amd import ops
    B, T = 1, 256
    print(f"\n[paired-gva] op={op} HV={HV} HQ={HQ}", flush=True)
    assert ops.paired_tile(B, HV, T // 64, GATE[op])
    xs, dO = make_inputs(op, B, T, HV, seed=53, gate="mild" if op in ("kda", "gdn2") else "default",
                         h0=op != "gdn2")
    if HQ != HV:
        xs["q"], xs["k"] = xs["q"][:, :, ::HV // HQ].contiguous(), xs["k"][:, :, ::HV // HQ].contiguous()
    dev = torch.device("cuda")
    kw = dict(disable_recompute=False) if op in ("kda", "gdn2") else {}

    def run():
        xg = {n: v.to(dev).requires_grad_() for n, v in xs.items()}
        with fdr.use_backend("optimized", ops=(op,)):
            o, ht = getattr(fdr, OPNAME[op])(**xg, output_final_state=True, **kw)
        outs = (o,) if op == "gdn2" else (o, ht)      # gdn2: no final-state gradient
        gouts = (dO.to(dev),) if op == "gdn2" else (dO.to(dev), torch.full_like(ht, 0.01))
        grads = torch.autograd.grad(outs, tuple(xg.values()), gouts)
        torch.cuda.synchronize()
        return grads

    calls = _count_pairs(monkeypatch)
    got = run()
    assert calls == ["one"], calls
    monkeypatch.setattr(ops, "PAIRED", False)
    off = run()
    for name, a, r in zip(xs, got, off):
        e = _rel(a, r)
        assert e <= 1e-5, (op, name, e)
