"""The recompute policy's side-by-side form (few heads, long rows): the forward scan
(fdr_fwd_h) enqueued on a second stream beside the segmented backward state recurrence
(fdr_state_bwd_segmented), the two being independent.  At B=1 H=8 T=8192 (the backend's
choice there, ops.side_by_side_pays), for the four families:

* the same gradients, bit for bit, as the same launches enqueued on one stream (the two
  streams change the order of execution only);
* against the direct kernels one after the other (pinned to the fp64 oracle elsewhere):
  rel-L2 <= 1e-2 per gradient, the two recurrence forms rounding their bf16 states at
  different points;
* captured in a HIP graph (fork / join of the side stream inside the capture) and replayed
  three times with eager work between the replays: every replay equals the eager call.
"""
import pytest
import torch

from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu

B, T, H = 1, 8192, 8


def _rel(a, r):
    a, r = a.double(), r.double()
    return float((a - r).norm() / r.norm().clamp_min(1e-30))


def _call(op):
    """The backward seam of `op` (recompute policy) on fixed inputs, as a closure."""
    from rewy_amd.backends import backward as bw
    from rewy_amd.hip_forward import chunk_forward_hip
    dev = torch.device("cuda")
    # long-memory gates for the vector families, so that the segment maps carry the state
    # across segments (with the default gates it decays to nothing within a chunk)
    xs, dO = make_inputs(op, B, T, H, seed=41, gate="mild" if op in ("kda", "gdn2") else "default")
    xs = {n: (None if v is None else v.to(dev)) for n, v in xs.items()}
    dO = dO.to(dev)
    _, _, sv = chunk_forward_hip(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"),
                                 b=xs.get("b"), w=xs.get("w"), initial_state=xs["initial_state"])
    dht = torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(3)).mul(0.1).to(dev)
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


@pytest.mark.parametrize("op", ["kda", "gdn2", "gdn", "delta"])
def test_side_by_side_recurrences(op, monkeypatch):
    from rewy_amd import ops
    from rewy_amd.backends import backward as bw
    print(f"\n[side-by-side] op={op} B={B} T={T} H={H}", flush=True)
    assert ops.side_by_side_pays(B, H, T // 64)
    run = _call(op)
    calls = []
    real = bw._side_by_side

    def spy(first, second):
        calls.append(1)
        return real(first, second)
    monkeypatch.setattr(bw, "_side_by_side", spy)
    got = [x.clone() for x in run()]
    torch.cuda.synchronize()
    assert calls, "the side-by-side form did not run"

    # the same launches on one stream
    monkeypatch.setattr(bw, "_side_by_side", lambda first, second: (first(), second()))
    one = run()
    torch.cuda.synchronize()
    for i, (a, r) in enumerate(zip(got, one)):
        assert torch.equal(a, r), (op, i)

    # the direct kernels one after the other
    monkeypatch.setattr(ops, "SIDE_BY_SIDE", False)
    monkeypatch.setattr(ops, "AFFINE_MAX_BH", -1)
    ref = run()
    torch.cuda.synchronize()
    for i, (a, r) in enumerate(zip(got, ref)):
        e = _rel(a, r)
        print(op, i, f"{e:.2e}", flush=True)
        assert e < 1e-2, (op, i, e)


@pytest.mark.parametrize("op", ["gdn", "kda"])
def test_side_by_side_under_graph_capture(op):
    from rewy_amd import ops
    print(f"\n[side-by-side graph] op={op} B={B} T={T} H={H}", flush=True)
    assert ops.side_by_side_pays(B, H, T // 64)
    run = _call(op)
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
        run()                     # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("op", ["kda", "gdn", "delta"])
def test_side_by_side_on_a_packed_batch(op, monkeypatch):
    """A skewed packed batch (sequences starting anywhere, one long, several short): the scan
    beside the direct state recurrence gives the gradients of the same launches on one stream,
    bit for bit."""
    from rewy_amd import ops
    from rewy_amd.backends import backward as bw
    from rewy_amd.hip_forward import chunk_forward_hip
    lens, H = [2048, 100, 300, 64, 577], 4
    T = sum(lens)
    print(f"\n[side-by-side packed] op={op} lens={lens} H={H}", flush=True)
    dev = torch.device("cuda")
    xs, dO = make_inputs(op, 1, T, H, seed=43)
    xs = {n: v.to(dev) for n, v in xs.items() if n != "initial_state"}
    dO = dO.to(dev)
    cu = torch.tensor([0] + lens).cumsum(0).to(dev)
    vl = ops.Varlen(cu, dev)
    assert not ops.fwd_h_wy_pays(vl.N, H, ops.GATE_VECTOR if op == "kda" else ops.GATE_SCALAR, vl)
    _, _, sv = chunk_forward_hip(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs["beta"], varlen=vl)
    common = dict(q=xs["q"], k=xs["k"], v=xs["v"], scale=sv["scale"], initial_state=None, do=dO, dht=None,
                  cu_seqlens=cu)
    if op == "kda":
        run = lambda: bw.kda_backward(beta=xs["beta"], Aqk=sv["Aqk"], Akk=sv["Akk"], g=sv["gc"], **common)[:5]
    elif op == "gdn":
        run = lambda: bw.gdn_backward(g=sv["gc"], beta=xs["beta"], A=sv["Akk"], **common)[:5]
    else:
        run = lambda: bw.delta_backward(beta=xs["beta"], A=sv["Akk"], **common)[:4]
    calls = []
    real = bw._side_by_side
    monkeypatch.setattr(bw, "_side_by_side", lambda a, b: (calls.append(1), real(a, b))[1])
    got = [x.clone() for x in run()]
    torch.cuda.synchronize()
    assert calls, "the side-by-side form did not run"
    monkeypatch.setattr(bw, "_side_by_side", lambda a, b: (a(), b()))
    one = run()
    torch.cuda.synchronize()
    for i, (a, r) in enumerate(zip(got, one)):
        assert torch.equal(a, r), (op, i)


@pytest.mark.parametrize("op", ["kda", "gdn"])
def test_side_by_side_with_grouped_heads_and_v_first_states(op, monkeypatch):
    """The side-by-side form with grouped value heads (q / k with 4 heads, 8 value heads) and
    V-first states: KDA takes it (its q / k head map is the prepare kernel's); GDN, whose
    segmented recurrence reads raw q / k per value head, keeps the direct kernels.  Both
    against the direct kernels one after the other (rel-L2 <= 1e-2 per gradient)."""
    from rewy_amd import ops
    from rewy_amd.backends import backward as bw
    from rewy_amd.hip_forward import chunk_forward_hip
    HV, G = 8, 2
    print(f"\n[side-by-side gva+vf] op={op} B={B} T={T} HV={HV} G={G}", flush=True)
    dev = torch.device("cuda")
    xs, dO = make_inputs(op, B, T, HV, seed=47)
    xs = {n: v.to(dev) for n, v in xs.items()}
    xs["q"] = xs["q"][:, :, ::G].contiguous()
    xs["k"] = xs["k"][:, :, 1::G].contiguous()
    h0 = xs["initial_state"].transpose(-1, -2).contiguous()           # [N, HV, V, K]
    dO = dO.to(dev)
    _, _, sv = chunk_forward_hip(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs["beta"], initial_state=h0,
                                 state_v_first=True)
    dht = torch.randn(B, HV, 128, 128, generator=torch.Generator().manual_seed(5)).mul(0.1).to(dev)
    common = dict(q=xs["q"], k=xs["k"], v=xs["v"], scale=sv["scale"], initial_state=h0, do=dO, dht=dht,
                  state_v_first=True)
    if op == "kda":
        run = lambda: bw.kda_backward(beta=xs["beta"], Aqk=sv["Aqk"], Akk=sv["Akk"], g=sv["gc"], **common)[:6]
    else:
        run = lambda: bw.gdn_backward(g=sv["gc"], beta=xs["beta"], A=sv["Akk"], **common)[:6]
    calls = []
    real = bw._side_by_side
    monkeypatch.setattr(bw, "_side_by_side", lambda a, b: (calls.append(1), real(a, b))[1])
    got = [x.clone() for x in run()]
    torch.cuda.synchronize()
    assert bool(calls) == (op == "kda"), calls
    monkeypatch.setattr(ops, "SIDE_BY_SIDE", False)
    monkeypatch.setattr(ops, "AFFINE_MAX_BH", -1)
    ref = run()
    torch.cuda.synchronize()
    for i, (a, r) in enumerate(zip(got, ref)):
        e = _rel(a, r)
        print(op, i, f"{e:.2e}", flush=True)
        assert e < 1e-2, (op, i, e)
