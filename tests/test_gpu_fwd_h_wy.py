"""fdr_fwd_h_wy (fdr_prepare_wu's w / u formed inside the fdr_fwd_h sweep, scalar / no gate)
against the two kernels it replaces, which tests/test_gpu_recompute.py holds to the fp64
oracle: w, h, v_new and the final state must be the same bits -- dense rows, every value-tile
width, an initial state in both layouts (state_v_first), grouped q / k heads, and packed
batches whose sequences start on chunk boundaries or anywhere.  One oracle check besides."""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu
GATE = {"delta": 0, "gdn": 1}


def _case(op, B, T, H, seed, qk_groups=1):
    from rewy_amd.forward import chunk_forward
    xs, _ = make_inputs(op, B, T, H, seed=seed)
    _, _, sv = chunk_forward(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"),
                             initial_state=xs["initial_state"])
    dev = torch.device("cuda")
    k = xs["k"][:, :, ::qk_groups] if qk_groups > 1 else xs["k"]
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    return dict(k=cu(k), v=cu(xs["v"]), A=cu(sv["Akk"]), g=cu(sv["gc"]) if op == "gdn" else None,
                beta=cu(xs["beta"]), h0=cu(xs["initial_state"])), xs, sv


def _both(op, a, vb=0, vf=False, varlen=None, h0=None):
    from rewy_amd import ops
    gate = GATE[op]
    pre = ops.prepare_wu(a["k"], a["v"], a["A"], gate, g=a["g"], beta=a["beta"], varlen=varlen)
    h, vn, ht = ops.fwd_h(a["k"], pre["w"], pre["u"], a["g"], gate, h0=h0, want_final=True, value_block=vb,
                          method="direct", varlen=varlen, state_v_first=vf)
    w2, h2, vn2, ht2 = ops.fwd_h_wy(a["k"], a["v"], a["A"], a["g"], gate, a["beta"], h0=h0, want_final=True,
                                    value_block=vb, varlen=varlen, state_v_first=vf)
    torch.cuda.synchronize()
    for n, x, y in (("w", pre["w"], w2), ("h", h, h2), ("v_new", vn, vn2), ("final", ht, ht2)):
        assert torch.equal(x, y), (n, float((x.float() - y.float()).abs().max()))


@pytest.mark.parametrize("op", ["gdn", "delta"])
@pytest.mark.parametrize("vb", [16, 32, 64])
def test_fwd_h_wy_equals_prepare_then_scan(op, vb):
    print(f"\n[fwd_h_wy] op={op} vb={vb}", flush=True)
    a, _, _ = _case(op, 2, 320, 3, seed=61)
    _both(op, a, vb=vb, h0=a["h0"])


@pytest.mark.parametrize("vf", [False, True])
def test_fwd_h_wy_state_layouts_and_grouped_heads(vf):
    print(f"\n[fwd_h_wy] gdn grouped heads, state_v_first={vf}", flush=True)
    a, _, _ = _case("gdn", 1, 256, 4, seed=62, qk_groups=2)
    h0 = a["h0"].transpose(-1, -2).contiguous() if vf else a["h0"]
    _both("gdn", a, vf=vf, h0=h0)


@pytest.mark.parametrize("lens", [[128, 64, 256], [100, 37, 0, 64, 1, 150]])
@pytest.mark.parametrize("op", ["gdn", "delta"])
def test_fwd_h_wy_packed(op, lens):
    from rewy_amd import ops
    print(f"\n[fwd_h_wy] packed op={op} lens={lens}", flush=True)
    T = sum(lens)
    a, _, _ = _case(op, 1, -(-T // 64) * 64, 2, seed=63)
    a = {n: (x[:, :T].contiguous() if x is not None and n != "h0" else x) for n, x in a.items()}
    dev = torch.device("cuda")
    vl = ops.Varlen(torch.tensor([0] + lens).cumsum(0), dev)
    h0 = (torch.randn(len(lens), 2, 128, 128, generator=torch.Generator().manual_seed(64)) * 0.05).to(dev)
    _both(op, a, varlen=vl, h0=h0)


def test_fwd_h_wy_against_the_oracle():
    from rewy_amd import ops
    print("\n[fwd_h_wy] gdn vs oracle", flush=True)
    a, xs, sv = _case("gdn", 2, 256, 2, seed=65)
    n = lambda x: None if x is None else x.double().numpy()
    ref = O.forward("gdn", n(xs["q"]), n(xs["k"]), n(xs["v"]), g=n(xs["g"]), beta=n(xs["beta"]),
                    h0=n(xs["initial_state"]))
    w, h, vn, ht = ops.fwd_h_wy(a["k"], a["v"], a["A"], a["g"], 1, a["beta"], h0=a["h0"], want_final=True)
    torch.cuda.synchronize()
    rel = lambda x, r: float(np.linalg.norm(n(x.cpu()) - r) / np.linalg.norm(r))
    e = dict(w=rel(w, ref["w"]), h=rel(h, ref["h"]), v_new=rel(vn, ref["v_new"]), final=rel(ht, ref["final"]))
    print("rel-L2 vs oracle", e, flush=True)
    assert max(e.values()) < 1e-2, e
