"""fdr_fwd_h_u (the forward scan forming u = Akk (beta v | w_gate v) itself) and fdr_prepare_wu
without u, the pair the paired recurrences run, against fdr_prepare_wu + fdr_fwd_h: w, qg, kg
of the two prepare modes and h, v_new, the final state of the two scans bit for bit (u is
formed with prepare_wu's MFMA sequence and roundings), for the four families, every tile
width, V-first states and grouped q / k heads."""
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
    d["Akk"], d["gc"] = cu(sv["Akk"]), cu(sv["gc"])
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
    ks = full["kg"] if vec else d["k"]
    for vf in (False, True):
        h0 = d["initial_state"].transpose(-1, -2).contiguous() if vf else d["initial_state"]
        ref = ops.fwd_h(ks, full["w"], full["u"], d["gc"], gate, h0=h0, want_final=True, value_block=vb,
                        method="direct", state_v_first=vf)
        got = ops.fwd_h_u(ks, part["w"], d["v"], d["Akk"], d["gc"], gate, beta=d.get("beta"), w_gate=d.get("w"),
                          h0=h0, want_final=True, value_block=vb, state_v_first=vf)
        torch.cuda.synchronize()
        for n, a, r in zip(("h", "v_new", "final"), got, ref):
            assert torch.equal(a, r), (op, vb, vf, n)


@pytest.mark.parametrize("op", ["gdn", "delta"])
def test_fwd_h_u_grouped_heads(op):
    from rewy_amd import ops
    B, T, H, HQ = 1, 192, 4, 2
    print(f"\n[fwd_h_u gva] op={op}", flush=True)
    d = _inputs(op, B, T, H, HQ, 72)
    gate = GATE[op]
    full = ops.prepare_wu(d["k"], d["v"], d["Akk"], gate, g=d["gc"], beta=d["beta"])
    part = ops.prepare_wu(d["k"], d["v"], d["Akk"], gate, g=d["gc"], beta=d["beta"], want_u=False)
    assert torch.equal(part["w"], full["w"])
    ref = ops.fwd_h(d["k"], full["w"], full["u"], d["gc"], gate, h0=d["initial_state"], method="direct")
    got = ops.fwd_h_u(d["k"], part["w"], d["v"], d["Akk"], d["gc"], gate, beta=d["beta"], h0=d["initial_state"])
    torch.cuda.synchronize()
    for n, a, r in zip(("h", "v_new"), got[:2], ref[:2]):
        assert torch.equal(a, r), (op, n)
