"""fdr_fwd_h_u (the forward scan forming u = Akk (beta v | w_gate v), and a vector gate's kg,
itself) and fdr_prepare_wu without u (and without qg / kg), the pair the paired recurrences
run, against fdr_prepare_wu + fdr_fwd_h: w, qg, kg of the prepare modes and h, v_new, the
final state of the two scans bit for bit (u and kg are formed with prepare_wu's MFMA sequence
and roundings), for the four families, every tile width, V-first states and grouped q / k
heads; and with w formed in the scan as well (w = NULL: no fdr_prepare_wu).  Likewise
fdr_state_bwd_raw_qk (qg / kg, and with w = NULL w, formed in the state recurrence) against
fdr_prepare_wu's qg / kg / w then fdr_state_bwd."""
import pytest
import torch

from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu

GATE = {"kda": 2, "gdn2": 2, "gdn": 1, "delta": 0}


def _inputs(op, B, T, H, HQ, seed):
    from rewy_amd.forward import chunk_forward
    xs, _ = make_inputs(op, B, T, H, seed=seed)
    _, _, sv = chunk_forward(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"), b=xs.get("b"),
                             w=xs.get("w"), initial_state=xs["initial_state"])
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    d = {n: cu(x) for n, x in xs.items()}
    d["Akk"], d["gc"], d["Aqk"] = cu(sv["Akk"]), cu(sv["gc"]), cu(sv.get("Aqk"))
    if HQ != H:
        d["q"], d["k"] = d["q"][:, :, ::H // HQ].contiguous(), d["k"][:, :, ::H // HQ].contiguous()
    return d


@pytest.mark.parametrize("vb", [16, 32, 64])
@pytest.mark.parametrize("op", ["kda", "gdn2", "gdn", "delta"])
def test_fwd_h_u_equals_prepare_then_fwd_h(op, vb):
    from rewy_amd import ops
    B, T, H = 2, 256, 3
    print(f"\n[fwd_h_u] op={op} value_block={vb}", flush=True)
    d = _inputs(op, B, T, H, H, 71)
    gate = GATE[op]
    vec = gate == 2
    kw = dict(g=d["gc"], beta=d.get("beta"), b=d.get("b"), w=d.get("w"), q=d["q"], want_qkg=vec)
    full = ops.prepare_wu(d["k"], d["v"], d["Akk"], gate, **kw)
    part = ops.prepare_wu(d["k"], d["v"], d["Akk"], gate, want_u=False, **kw)
    for n in ("w", "qg", "kg"):
        if full[n] is not None:
            assert torch.equal(part[n], full[n]), n
    assert part["u"] is None
    if vec:         # w only
        bare = ops.prepare_wu(d["k"], d["v"], d["Akk"], gate, want_u=False, **dict(kw, want_qkg=False))
        assert bare["qg"] is None and bare["kg"] is None and bare["u"] is None
        assert torch.equal(bare["w"], full["w"])
    ks = full["kg"] if vec else d["k"]
    for vf in (False, True):
        h0 = d["initial_state"].transpose(-1, -2).contiguous() if vf else d["initial_state"]
        ref = ops.fwd_h(ks, full["w"], full["u"], d["gc"], gate, h0=h0, want_final=True, value_block=vb,
                        method="direct", state_v_first=vf)
        got = ops.fwd_h_u(d["k"], part["w"], d["v"], d["Akk"], d["gc"], gate, beta=d.get("beta"),
                          w_gate=d.get("w"), h0=h0, want_final=True, value_block=vb, state_v_first=vf)
        torch.cuda.synchronize()
        for n, a, r in zip(("h", "v_new", "final"), got, ref):
            assert torch.equal(a, r), (op, vb, vf, n)
        if vec:     # kg read as prepare_wu wrote it
            got = ops.fwd_h_u(d["k"], part["w"], d["v"], d["Akk"], d["gc"], gate, beta=d.get("beta"),
                              w_gate=d.get("w"), h0=h0, want_final=True, value_block=vb, state_v_first=vf,
                              kg=full["kg"])
            torch.cuda.synchronize()
            for n, a, r in zip(("h", "v_new", "final"), got, ref):
                assert torch.equal(a, r), (op, vb, vf, "kg read", n)
        # w formed in the scan too (no prepare_wu)
        got = ops.fwd_h_u(d["k"], None, d["v"], d["Akk"], d["gc"], gate, beta=d.get("beta"), w_gate=d.get("w"),
                          b=d.get("b"), h0=h0, want_final=True, value_block=vb, state_v_first=vf)
        torch.cuda.synchronize()
        for n, a, r in zip(("h", "v_new", "final"), got, ref):
            assert torch.equal(a, r), (op, vb, vf, "w formed", n)


@pytest.mark.parametrize("op", ["kda", "gdn", "delta"])
def test_fwd_h_u_grouped_heads(op):
    from rewy_amd import ops
    B, T, H, HQ = 1, 192, 4, 2
    print(f"\n[fwd_h_u gva] op={op}", flush=True)
    d = _inputs(op, B, T, H, HQ, 72)
    gate = GATE[op]
    vec = gate == 2
    full = ops.prepare_wu(d["k"], d["v"], d["Akk"], gate, g=d["gc"], beta=d["beta"], q=d["q"], want_qkg=vec)
    part = ops.prepare_wu(d["k"], d["v"], d["Akk"], gate, g=d["gc"], beta=d["beta"], want_u=False)
    assert torch.equal(part["w"], full["w"])
    ref = ops.fwd_h(full["kg"] if vec else d["k"], full["w"], full["u"], d["gc"], gate, h0=d["initial_state"],
                    method="direct")
    for w in (part["w"], None):
        got = ops.fwd_h_u(d["k"], w, d["v"], d["Akk"], d["gc"], gate, beta=d["beta"], h0=d["initial_state"])
        torch.cuda.synchronize()
        for n, a, r in zip(("h", "v_new"), got[:2], ref[:2]):
            assert torch.equal(a, r), (op, w is None, n)


@pytest.mark.parametrize("vb", [16, 32, 64])
@pytest.mark.parametrize("op,HQ", [("kda", 3), ("gdn2", 3), ("kda", 1)])
def test_state_bwd_raw_qk_equals_prepared_qg_kg(op, HQ, vb):
    from rewy_amd import ops
    B, T, H = 2, 256, 3
    print(f"\n[state raw_qk] op={op} HQ={HQ} value_block={vb}", flush=True)
    d = _inputs(op, B, T, H, HQ, 73)
    pre = ops.prepare_wu(d["k"], d["v"], d["Akk"], 2, g=d["gc"], beta=d.get("beta"), b=d.get("b"), w=d.get("w"),
                         q=d["q"], want_qkg=True)
    gen = torch.Generator().manual_seed(74)
    dev = torch.device("cuda")
    dO = torch.randn(B, T, H, 128, generator=gen).to(dev, torch.bfloat16)
    dht = (torch.randn(B, H, 128, 128, generator=gen) * 0.1).to(dev)
    for vf in (False, True):
        common = dict(aqk=d["Aqk"], dht=dht, want_dh0=True, value_block=vb, method="direct", state_v_first=vf)
        ref = ops.state_bwd(pre["qg"], pre["kg"], pre["w"], d["gc"], 2, dO, 0.088, **common)
        got = ops.state_bwd(d["q"], d["k"], pre["w"], d["gc"], 2, dO, 0.088, raw_qk=True, **common)
        formed = ops.state_bwd(d["q"], d["k"], None, d["gc"], 2, dO, 0.088, raw_qk=True, beta=d.get("beta"),
                               b=d.get("b"), Akk=d["Akk"], **common)
        torch.cuda.synchronize()
        for n, a, f, r in zip(("dh", "dR", "dh0"), got, formed, ref):
            assert torch.equal(a, r), (op, HQ, vb, vf, n)
            assert torch.equal(f, r), (op, HQ, vb, vf, "w formed", n)
