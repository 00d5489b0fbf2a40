"""The KDA chunk kernel with the in-kernel gate's backward folded into its dg stores
(fdr_chunk_bwd_gate_fold) against the two-pass path it replaces: fdr_chunk_bwd, then
fdr_kda_gate_bwd on its dg (both pinned elsewhere against the oracle and fp64 autograd).
Same fp32 arithmetic both ways: dq/dk/dv/dbeta bit-for-bit up to 1e-6 rel-L2, dg_raw
1e-5 (fp32) or 4e-3 (bf16 output rounding), dA_log / ddt_bias 1e-5 (summed in another
order)."""
import pytest
import torch

from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu


def _rel(a, r):
    a, r = a.double().cpu(), r.double().cpu()
    return float((a - r).norm() / r.norm().clamp_min(1e-30))


@pytest.mark.parametrize("mode", ["softplus", "bounded", "bounded_no_A"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,with_bias", [((1, 128, 2), True), ((2, 192, 3), True), ((1, 512, 20), True),
                                              ((2, 192, 3), False)])
def test_gate_fold_matches_two_pass(mode, dtype, shape, with_bias):
    from rewy_amd import ops
    from rewy_amd.forward import chunk_forward
    from rewy_amd.gates import kda_gate_bwd
    B, T, H = shape
    print(f"\n[gate-fold] mode={mode} dtype={dtype} shape={shape} bias={with_bias}", flush=True)
    xs, dO = make_inputs("kda", B, T, H, seed=17)
    _, _, sv = chunk_forward("kda", xs["q"], xs["k"], xs["v"], g=xs["g"], beta=xs["beta"],
                             initial_state=xs["initial_state"])
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    gen = torch.Generator().manual_seed(4)
    g_raw = (torch.randn(B, T, H, 128, generator=gen) * 3).to(dtype).to(dev)
    A = None if mode == "bounded_no_A" else (torch.randn(H, generator=gen) * 0.5).to(dev)
    dt = (torch.randn(H * 128, generator=gen) * 0.5).to(dev) if with_bias else None
    lb = None if mode == "softplus" else -5.0
    scale = sv["scale"]
    gc = cu(sv["gc"])
    dh, dR, _ = ops.state_bwd(cu(sv["qg"]), cu(sv["kg"]), cu(sv["w"]), gc, ops.GATE_VECTOR, cu(dO), scale,
                              aqk=cu(sv["Aqk"]))
    args = (cu(xs["q"]), cu(xs["k"]), cu(xs["v"]), cu(sv["v_new"]), cu(dO), dR, gc, ops.GATE_VECTOR,
            cu(sv["Akk"]), cu(sv["h"]), dh, scale)
    ref = ops.chunk_bwd(*args, beta=cu(xs["beta"]))
    r_raw, r_A, r_dt = kda_gate_bwd(ref["dg"], g_raw, A, dt, lb, native=True)
    got = ops.chunk_bwd(*args, beta=cu(xs["beta"]),
                        gate_fold=dict(g_raw=g_raw, A_log=A, dt_bias=dt, lower_bound=lb))
    torch.cuda.synchronize()
    for name in ("dq", "dk", "dv", "dbeta"):
        assert _rel(got[name], ref[name]) < 1e-6, (name, _rel(got[name], ref[name]))
    assert got["dg"].dtype == dtype
    tol = 1e-5 if dtype == torch.float32 else 4e-3
    assert _rel(got["dg"], r_raw) < tol, _rel(got["dg"], r_raw)
    assert (got["dA_log"] is None) == (r_A is None)
    if r_A is not None:
        assert _rel(got["dA_log"], r_A) < 1e-5, _rel(got["dA_log"], r_A)
    assert (got["ddt_bias"] is None) == (r_dt is None)
    if r_dt is not None:
        assert _rel(got["ddt_bias"], r_dt) < 1e-5, _rel(got["ddt_bias"], r_dt)
    # a second call reuses nothing stale: the partial sums are rewritten, not accumulated
    again = ops.chunk_bwd(*args, beta=cu(xs["beta"]),
                          gate_fold=dict(g_raw=g_raw, A_log=A, dt_bias=dt, lower_bound=lb))
    torch.cuda.synchronize()
    assert torch.equal(again["dg"], got["dg"])
    if r_dt is not None:
        assert torch.equal(again["ddt_bias"], got["ddt_bias"])
