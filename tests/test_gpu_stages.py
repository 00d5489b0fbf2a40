"""Stage parity of the HIP kernels against the fp64 oracle's stage functions.

Inputs come from the package's torch forward (run on the CPU), are rounded to
the dtypes the kernels consume, and are handed to both the kernel (through the
C-ABI) and the oracle as the same values.  Tolerances: rel-L2 per tensor, with
bf16 outputs (dh, dR, dq, dk, dv) at 1e-2 and fp32 outputs at 5e-3.
"""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu

GATE = {"delta": 0, "gdn": 1, "kda": 2, "gdn2": 2}


def _np(x):
    return x.detach().double().cpu().numpy()


def _rel(a, r):
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    return float(np.linalg.norm(a - r) / max(np.linalg.norm(r), 1e-30))


def _setup(op, B, T, H, seed, **kw):
    from rewy_amd.forward import chunk_forward
    xs, dO = make_inputs(op, B, T, H, seed=seed, **kw)
    _, _, sv = chunk_forward(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"),
                             b=xs.get("b"), w=xs.get("w"), initial_state=xs.get("initial_state"))
    return xs, dO, sv


CASES = [(op, shp, "default", 0) for op in ("kda", "gdn", "delta", "gdn2") for shp in ((1, 128, 2), (2, 256, 3))]
CASES += [("kda", (1, 192, 2), "wide", 5), ("gdn2", (1, 192, 2), "wide", 0), ("gdn", (1, 128, 2), "default", 3)]
# more chunk-heads than the GPU has CUs: the persistent scalar/no-gate chunk kernel walks
# 1 or 2 chunk-heads per work-group (300 is not a multiple of the CU count)
CASES += [("gdn", (1, 64 * 300, 1), "default", 7), ("delta", (2, 64 * 150, 1), "default", 0)]


@pytest.mark.parametrize("op,shape,gate,bz", CASES)
def test_state_and_chunk_kernels(op, shape, gate, bz):
    from rewy_amd import ops
    B, T, H = shape
    print(f"\n[stage] op={op} B={B} T={T} H={H} gate={gate} beta_zero_every={bz}", flush=True)
    xs, dO, sv = _setup(op, B, T, H, seed=11, gate=gate, beta_zero_every=bz)
    dev = torch.device("cuda")
    scale = sv["scale"]
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    gc = sv["gc"]
    if op in ("kda", "gdn2"):
        qs, ks = sv["qg"], sv["kg"]
    else:
        qs, ks = xs["q"], xs["k"]
    dht = torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(3)) * 0.1
    dh, dR, dh0 = ops.state_bwd(cu(qs), cu(ks), cu(sv["w"]), cu(gc), GATE[op], cu(dO), scale,
                                aqk=cu(sv["Aqk"]), dht=cu(dht))
    torch.cuda.synchronize()
    # oracle: gated q/k for the scalar families are formed in fp64 from raw q/k
    if op in ("kda", "gdn2"):
        oq, ok_, og = _np(qs), _np(ks), _np(gc)
    else:
        gcn = np.zeros((B, T, H)) if gc is None else _np(gc)
        G = O._to_chunks(gcn[..., None], 64)
        gam = np.exp2(G)
        kdec = np.exp2(G[..., -1:, :] - G)
        oq = O._from_chunks(O._to_chunks(_np(xs["q"]), 64) * gam)
        ok_ = O._from_chunks(O._to_chunks(_np(xs["k"]), 64) * kdec)
        og = np.broadcast_to(gcn[..., None], (B, T, H, 128))
    odv = O.dv_local(_np(sv["Aqk"]), _np(dO))
    rdh, rdR, rdh0 = O.stage_state_bwd(oq, ok_, _np(sv["w"]), og, _np(dO), odv, dht=_np(dht), scale=scale)
    e = dict(dh=_rel(_np(dh), rdh), dR=_rel(_np(dR), rdR), dh0=_rel(_np(dh0), rdh0))
    print("state", e, flush=True)
    assert e["dh"] < 1e-2 and e["dR"] < 1e-2 and e["dh0"] < 5e-3, e

    out = ops.chunk_bwd(cu(xs["q"]), cu(xs["k"]), cu(xs["v"]), cu(sv["v_new"]), cu(dO), dR,
                        cu(gc), GATE[op], cu(sv["Akk"]), cu(sv["h"]), dh, scale,
                        beta=cu(xs.get("beta")), b=cu(xs.get("b")), w=cu(xs.get("w")))
    torch.cuda.synchronize()
    ref = O.stage_post(op, _np(xs["q"]), _np(xs["k"]), _np(xs["v"]), None if gc is None else _np(gc),
                       beta=None if "beta" not in xs else _np(xs["beta"]),
                       b=None if "b" not in xs else _np(xs["b"]), w=None if "w" not in xs else _np(xs["w"]),
                       Akk=_np(sv["Akk"]), h=_np(sv["h"]), dh=_np(dh), v_new=_np(sv["v_new"]),
                       dO=_np(dO), dR=_np(dR), scale=scale)
    errs = {}
    for name in ("dq", "dk", "dv", "dg", "dbeta", "db", "dw"):
        if name in ref:
            errs[name] = _rel(_np(out[name]), ref[name])
    print("chunk", errs, flush=True)
    for name, e_ in errs.items():
        assert np.isfinite(_np(out[name])).all(), name
        assert e_ < (1e-2 if name in ("dq", "dk", "dv", "db", "dw") else 5e-3), (name, errs)


@pytest.mark.parametrize("op", ["kda", "gdn", "delta"])
@pytest.mark.parametrize("vb", [16, 32, 64])
def test_state_kernel_value_blocks(op, vb):
    """Every value-tile width of the direct state kernel (the default picks it from B*H;
    32-wide tiles run 16 waves, the others 8) against the oracle."""
    from rewy_amd import ops
    B, T, H = 1, 256, 2
    print(f"\n[state vb] op={op} value_block={vb}", flush=True)
    xs, dO, sv = _setup(op, B, T, H, seed=41)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    gc = sv["gc"]
    if op == "kda":
        qs, ks, oq, ok_, og = sv["qg"], sv["kg"], _np(sv["qg"]), _np(sv["kg"]), _np(gc)
    else:
        qs, ks = xs["q"], xs["k"]
        gcn = np.zeros((B, T, H)) if gc is None else _np(gc)
        G = O._to_chunks(gcn[..., None], 64)
        oq = O._from_chunks(O._to_chunks(_np(xs["q"]), 64) * np.exp2(G))
        ok_ = O._from_chunks(O._to_chunks(_np(xs["k"]), 64) * np.exp2(G[..., -1:, :] - G))
        og = np.broadcast_to(gcn[..., None], (B, T, H, 128))
    dht = torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(4)) * 0.1
    dh, dR, dh0 = ops.state_bwd(cu(qs), cu(ks), cu(sv["w"]), cu(gc), GATE[op], cu(dO), sv["scale"],
                                aqk=cu(sv["Aqk"]), dht=cu(dht), value_block=vb, method="direct")
    torch.cuda.synchronize()
    odv = O.dv_local(_np(sv["Aqk"]), _np(dO))
    rdh, rdR, rdh0 = O.stage_state_bwd(oq, ok_, _np(sv["w"]), og, _np(dO), odv, dht=_np(dht), scale=sv["scale"])
    e = dict(dh=_rel(_np(dh), rdh), dR=_rel(_np(dR), rdR), dh0=_rel(_np(dh0), rdh0))
    print("state", e, flush=True)
    assert e["dh"] < 1e-2 and e["dR"] < 1e-2 and e["dh0"] < 5e-3, e
