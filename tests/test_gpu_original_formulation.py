"""The chunk kernel in the original 7-product formulation (fdr_chunk_bwd_original, the
same-GPU comparator of the residual one) against the fp64 oracle's stage function and
against the residual kernel on the same inputs.

The oracle's stage function computes the chunk-stage gradients from the closed form
(pinned by complex step against the token recurrence), independently of which product
list forms them, so both formulations must meet it; tolerances as for the residual kernel
(rel-L2 1e-2 for bf16 outputs, 5e-3 for fp32).  Cases: the BASELINE gate distribution, rows
with beta = 0 (dbeta's direct VJP is the original's rule on every row), wide gate spans
(the pairwise intra diagonal), several chunks and heads.
"""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests.test_gpu_stages import _np, _rel, _setup

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,gate,bz", [((1, 128, 2), "default", 0), ((2, 256, 3), "default", 5),
                                            ((1, 192, 2), "wide", 0)])
def test_original_formulation_matches_oracle_and_residual(shape, gate, bz):
    from rewy_amd import ops
    B, T, H = shape
    print(f"\n[original] shape={shape} gate={gate} beta_zero_every={bz}", flush=True)
    xs, dO, sv = _setup("kda", B, T, H, seed=19, gate=gate, beta_zero_every=bz)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    scale = sv["scale"]
    gc = cu(sv["gc"])
    dh, dR, _ = ops.state_bwd(cu(sv["qg"]), cu(sv["kg"]), cu(sv["w"]), gc, 2, cu(dO), scale, aqk=cu(sv["Aqk"]))
    args = (cu(xs["q"]), cu(xs["k"]), cu(xs["v"]), cu(sv["v_new"]), cu(dO), dR, gc)
    orig = ops.chunk_bwd_original(*args, cu(sv["Akk"]), cu(sv["h"]), dh, scale, cu(xs["beta"]))
    resid = ops.chunk_bwd(*args, 2, cu(sv["Akk"]), cu(sv["h"]), dh, scale, beta=cu(xs["beta"]))
    torch.cuda.synchronize()
    ref = O.stage_post("kda", _np(xs["q"]), _np(xs["k"]), _np(xs["v"]), _np(sv["gc"]), beta=_np(xs["beta"]),
                       Akk=_np(sv["Akk"]), h=_np(sv["h"]), dh=_np(dh), v_new=_np(sv["v_new"]), dO=_np(dO),
                       dR=_np(dR), scale=scale)
    e_o = {n: _rel(_np(orig[n]), ref[n]) for n in ("dq", "dk", "dv", "dg", "dbeta")}
    e_r = {n: _rel(_np(orig[n]), _np(resid[n])) for n in ("dq", "dk", "dv", "dg", "dbeta")}
    print("original vs oracle", e_o, "vs residual", e_r, flush=True)
    for n, e in e_o.items():
        assert np.isfinite(_np(orig[n])).all(), n
        assert e < (1e-2 if n in ("dq", "dk", "dv") else 5e-3), (n, e_o)
    for n, e in e_r.items():
        assert e < (1e-2 if n in ("dq", "dk", "dv") else 5e-3), (n, e_r)
