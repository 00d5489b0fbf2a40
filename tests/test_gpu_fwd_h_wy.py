"""fdr_fwd_h_wy (fdr_prepare_wu's w / u formed inside the fdr_fwd_h sweep) against the two
kernels it replaces, which tests/test_gpu_recompute.py holds to the fp64 oracle: w (and for
the vector gates qg, kg), h, v_new and the final state must be the same bits -- all four
families, dense rows, every value-tile width, an initial state in both layouts
(state_v_first), grouped q / k heads, and packed batches whose sequences start on chunk
boundaries or anywhere.  One oracle check besides."""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu
GATE = {"delta": 0, "gdn": 1, "kda": 2, "gdn2": 2}


def _case(op, B, T, H, seed, qk_groups=1):
    from rewy_amd.forward import chunk_forward
    xs, _ = make_inputs(op, B, T, H, seed=seed)
    _, _, sv = chunk_forward(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"), b=xs.get("b"),
                             w=xs.get("w"), initial_state=xs["initial_state"])
    dev = torch.device("cuda")
    sub = (lambda x: x[:, :, ::qk_groups]) if qk_groups > 1 else (lambda x: x)
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    return dict(q=cu(sub(xs["q"])), k=cu(sub(xs["k"])), v=cu(xs["v"]), A=cu(sv["Akk"]),
                g=cu(sv["gc"]) if op != "delta" else None, beta=cu(xs.get("beta")), b=cu(xs.get("b")),
                w=cu(xs.get("w")), h0=cu(xs["initial_state"])), xs, sv


def _both(op, a, vb=0, vf=False, varlen=None, h0=None):
    from rewy_amd import ops
    gate = GATE[op]
    vec = gate == 2
    q = a["q"] if vec else None
    pre = ops.prepare_wu(a["k"], a["v"], a["A"], gate, g=a["g"], beta=a["beta"], b=a["b"], w=a["w"], q=q,
                         want_qkg=vec, varlen=varlen)
    h, vn, ht = ops.fwd_h(pre["kg"] if vec else a["k"], pre["w"], pre["u"], a["g"], gate, h0=h0, want_final=True,
                          value_block=vb, method="direct", varlen=varlen, state_v_first=vf)
    r = ops.fwd_h_wy(a["k"], a["v"], a["A"], a["g"], gate, beta=a["beta"], q=q, b=a["b"], w=a["w"], h0=h0,
                     want_final=True, value_block=vb, varlen=varlen, state_v_first=vf)
    torch.cuda.synchronize()
    pairs = [("w", pre["w"], r["w"]), ("h", h, r["h"]), ("v_new", vn, r["v_new"]), ("final", ht, r["final"])]
    if vec:
        pairs += [("qg", pre["qg"], r["qg"]), ("kg", pre["kg"], r["kg"])]
    for n, x, y in pairs:
        assert torch.equal(x, y), (n, float((x.float() - y.float()).abs().max()))


@pytest.mark.parametrize("op", ["gdn", "delta", "kda", "gdn2"])
@pytest.mark.parametrize("vb", [16, 32, 64])
def test_fwd_h_wy_equals_prepare_then_scan(op, vb):
    print(f"\n[fwd_h_wy] op={op} vb={vb}", flush=True)
    a, _, _ = _case(op, 2, 320, 3, seed=61)
    _both(op, a, vb=vb, h0=a["h0"])


@pytest.mark.parametrize("op", ["gdn", "kda"])
@pytest.mark.parametrize("vf", [False, True])
def test_fwd_h_wy_state_layouts_and_grouped_heads(op, vf):
    print(f"\n[fwd_h_wy] {op} grouped heads, state_v_first={vf}", flush=True)
    a, _, _ = _case(op, 1, 256, 4, seed=62, qk_groups=2)
    h0 = a["h0"].transpose(-1, -2).contiguous() if vf else a["h0"]
    _both(op, a, vf=vf, h0=h0)


@pytest.mark.parametrize("vb", [0, 64])
@pytest.mark.parametrize("lens", [[128, 64, 256], [100, 37, 0, 64, 1, 150]])
@pytest.mark.parametrize("op", ["gdn", "delta", "kda", "gdn2"])
def test_fwd_h_wy_packed(op, lens, vb):
    """gc and Akk from the HIP forward of the packed batch itself (per-sequence chunk-local
    gate cumsums: a vector gate's 2^(g_last - g) is bounded only then)"""
    from rewy_amd import ops
    from rewy_amd.hip_forward import chunk_forward_hip
    print(f"\n[fwd_h_wy] packed op={op} lens={lens} vb={vb}", flush=True)
    T = sum(lens)
    dev = torch.device("cuda")
    xs, _ = make_inputs(op, 1, T, 2, seed=63)
    xs = {n: x.to(dev) for n, x in xs.items() if n != "initial_state"}
    vl = ops.Varlen(torch.tensor([0] + lens).cumsum(0), dev)
    _, _, sv = chunk_forward_hip(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"), b=xs.get("b"),
                                 w=xs.get("w"), varlen=vl)
    a = dict(q=xs["q"], k=xs["k"], v=xs["v"], A=sv["Akk"], g=sv["gc"] if op != "delta" else None,
             beta=xs.get("beta"), b=xs.get("b"), w=xs.get("w"))
    h0 = (torch.randn(len(lens), 2, 128, 128, generator=torch.Generator().manual_seed(64)) * 0.05).to(dev)
    _both(op, a, vb=vb, varlen=vl, h0=h0)


def test_fwd_h_wy_against_the_oracle():
    from rewy_amd import ops
    print("\n[fwd_h_wy] gdn vs oracle", flush=True)
    a, xs, sv = _case("gdn", 2, 256, 2, seed=65)
    n = lambda x: None if x is None else x.double().numpy()
    ref = O.forward("gdn", n(xs["q"]), n(xs["k"]), n(xs["v"]), g=n(xs["g"]), beta=n(xs["beta"]),
                    h0=n(xs["initial_state"]))
    r = ops.fwd_h_wy(a["k"], a["v"], a["A"], a["g"], 1, beta=a["beta"], h0=a["h0"], want_final=True)
    w, h, vn, ht = r["w"], r["h"], r["v_new"], r["final"]
    torch.cuda.synchronize()
    rel = lambda x, r: float(np.linalg.norm(n(x.cpu()) - r) / np.linalg.norm(r))
    e = dict(w=rel(w, ref["w"]), h=rel(h, ref["h"]), v_new=rel(vn, ref["v_new"]), final=rel(ht, ref["final"]))
    print("rel-L2 vs oracle", e, flush=True)
    assert max(e.values()) < 1e-2, e


@pytest.mark.parametrize("op", ["kda", "gdn2"])
def test_recompute_backward_equals_full_saving(op):
    """B*H = 128 (64-wide value tiles): the vector-gate recompute policy takes fdr_fwd_h_wy,
    whose w, qg, kg, h, v_new are the bits the HIP forward saves (fdr_prepare_wu + fdr_fwd_h),
    so every gradient equals the full-saving backward's exactly."""
    from rewy_amd import ops
    from rewy_amd.backends import backward as bw
    from rewy_amd.hip_forward import chunk_forward_hip
    B, T, H = 8, 128, 16
    assert ops.fwd_h_wy_pays(B, H, ops.GATE_VECTOR)
    print(f"\n[fwd_h_wy] {op} recompute vs full saving B={B} T={T} H={H}", flush=True)
    dev = torch.device("cuda")
    xs, dO = make_inputs(op, B, T, H, seed=66)
    xs = {n: x.to(dev) for n, x in xs.items()}
    dO = dO.to(dev)
    _, _, sv = chunk_forward_hip(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"), b=xs.get("b"),
                                 w=xs.get("w"), initial_state=xs["initial_state"])
    common = dict(q=xs["q"], k=xs["k"], v=xs["v"], scale=sv["scale"], initial_state=xs["initial_state"], do=dO,
                  dht=None, g=sv["gc"], Aqk=sv["Aqk"], Akk=sv["Akk"])
    if op == "kda":
        run = lambda **kept: bw.kda_backward(beta=xs["beta"], **common, **kept)[:6]
        full = run(w=sv["w"], u=sv["u"], qg=sv["qg"], kg=sv["kg"], v_new=sv["v_new"], h=sv["h"])
    else:
        run = lambda **kept: bw.gdn2_backward(b=xs["b"], w_gate=xs["w"], **common, **kept)[:7]
        full = run(w_wy=sv["w"], u_wy=sv["u"], qg=sv["qg"], kg=sv["kg"], v_new=sv["v_new"], h=sv["h"])
    rec = run()
    torch.cuda.synchronize()
    for i, (a, r) in enumerate(zip(rec, full)):
        if r is None:
            assert a is None
            continue
        assert torch.equal(a, r), (i, float((a.float() - r.float()).abs().max()))


@pytest.mark.parametrize("op", ["gdn", "kda", "gdn2"])
def test_hip_forward_fused_scan_equals_the_pair(op):
    """The HIP forward with steps 2-3 as one sweep (fdr_fwd_h_wy) against the same forward with
    fdr_prepare_wu + fdr_fwd_h: o, the final state and every saved tensor but u, bit for bit"""
    from rewy_amd.hip_forward import chunk_forward_hip
    B, T, H = 8, 128, 16
    print(f"\n[fwd_h_wy] HIP forward {op} fused vs pair", flush=True)
    dev = torch.device("cuda")
    xs, _ = make_inputs(op, B, T, H, seed=67)
    xs = {n: x.to(dev) for n, x in xs.items()}
    run = lambda fuse: chunk_forward_hip(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"),
                                         b=xs.get("b"), w=xs.get("w"), initial_state=xs["initial_state"],
                                         output_final_state=True, fuse_scan=fuse)
    o1, f1, s1 = run(True)
    o0, f0, s0 = run(False)
    torch.cuda.synchronize()
    assert s1["u"] is None
    assert torch.equal(o1, o0) and torch.equal(f1, f0)
    for n in ("w", "qg", "kg", "h", "v_new"):
        if s0[n] is not None:
            assert torch.equal(s1[n], s0[n]), n
