"""Parity of the segmented state recurrence (fdr_state_bwd_segmented: per-segment affine
maps P, Q in parallel, a sequential chain over segments, every segment rerun from its
end state) with the fp64 oracle's stage function and with the direct kernel on the same
inputs.

Cases: every gate mode, segment counts that divide the chunk count and that do not
(uneven segments), one segment (the chain is a single step) and one chunk per segment,
two batch rows (segments never cross a row), a given and an absent dht, dh0 wanted and
not, dv_local given instead of Aqk, and every value-tile width of the rerun.  Tolerances
as for the direct kernel: rel-L2 1e-2 for bf16 outputs (dh, dR), 5e-3 for fp32 (dh0).
"""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests.test_gpu_affine import _gated
from tests.test_gpu_stages import GATE, _np, _rel, _setup

pytestmark = pytest.mark.gpu

CASES = [
    ("kda", (1, 64 * 24, 2), 4, 0, "aqk", True),
    ("kda", (2, 64 * 10, 2), 3, 16, "aqk", True),       # 10 chunks in 3 segments: 3, 3, 4
    ("gdn", (2, 64 * 9, 1), 9, 32, "aqk", False),      # one chunk per segment
    ("delta", (1, 64 * 7, 3), 1, 64, "aqk", True),     # a single segment
    ("gdn2", (1, 64 * 16, 2), 5, 0, "dv", True),
    ("kda", (1, 64 * 300, 1), 0, 0, "aqk", True),      # the automatic segment count
]


@pytest.mark.parametrize("op,shape,segs,vb,dv_from,with_dht", CASES)
def test_segmented_state_bwd(op, shape, segs, vb, dv_from, with_dht):
    from rewy_amd import ops
    B, T, H = shape
    print(f"\n[segmented] op={op} B={B} T={T} H={H} segments={segs} value_block={vb} dv={dv_from} "
          f"dht={with_dht}", flush=True)
    xs, dO, sv = _setup(op, B, T, H, seed=41)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    scale = sv["scale"]
    qs, ks, oq, ok_, og = _gated(op, xs, sv, B, T, H)
    odv = O.dv_local(_np(sv["Aqk"]), _np(dO))
    dht = torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(6)) * 0.1 if with_dht else None
    kw = dict(aqk=cu(sv["Aqk"])) if dv_from == "aqk" else dict(dv=cu(torch.from_numpy(odv).bfloat16()))
    args = (cu(qs), cu(ks), cu(sv["w"]), cu(sv["gc"]), GATE[op], cu(dO), scale)
    dh, dR, dh0 = ops.state_bwd(*args, dht=cu(dht), value_block=vb, method="segmented", segments=segs, **kw)
    ddh, ddR, ddh0 = ops.state_bwd(*args, dht=cu(dht), method="direct", **kw)
    _, _, none0 = ops.state_bwd(*args, dht=cu(dht), want_dh0=False, method="segmented", segments=segs, **kw)
    torch.cuda.synchronize()
    assert none0 is None
    odv_in = odv if dv_from == "aqk" else _np(kw["dv"])
    rdh, rdR, rdh0 = O.stage_state_bwd(oq, ok_, _np(sv["w"]), og, _np(dO), odv_in,
                                       dht=None if dht is None else _np(dht), scale=scale)
    e = dict(dh=_rel(_np(dh), rdh), dR=_rel(_np(dR), rdR), dh0=_rel(_np(dh0), rdh0))
    d = dict(dh=_rel(_np(dh), _np(ddh)), dR=_rel(_np(dR), _np(ddR)), dh0=_rel(_np(dh0), _np(ddh0)))
    print("vs oracle", e, "vs direct", d, flush=True)
    assert e["dh"] < 1e-2 and e["dR"] < 1e-2 and e["dh0"] < 5e-3, e
    assert d["dh"] < 1e-2 and d["dR"] < 1e-2 and d["dh0"] < 5e-3, d

