"""KDA's fused gate (use_gate_in_kernel): the explicit backward against fp64
autograd of the documented activations, and the public operator's wiring on the
CPU (original backend) against the same operator fed the activated gate.

Parity against FLA's own fused kernel is unpinned (FLA is not part of this
build); the activations are the ones the reference documents at
_compat/kda.py:250-294."""
import pytest
import torch

from rewy_amd.gates import kda_gate, kda_gate_bwd
from tests._inputs import make_inputs

FORMS = [(None, True, True), (None, True, False), (-5.0, True, True), (-5.0, False, True), (-3.0, True, False)]


@pytest.mark.parametrize("lower_bound,use_a,use_dt", FORMS)
def test_gate_backward_matches_autograd(lower_bound, use_a, use_dt):
    gen = torch.Generator().manual_seed(7)
    B, T, H, K = 2, 8, 3, 4
    g = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64, requires_grad=True)
    A = torch.randn(H, generator=gen, dtype=torch.float64, requires_grad=True) if use_a else None
    dt = torch.randn(H * K, generator=gen, dtype=torch.float64, requires_grad=True) if use_dt else None
    y = kda_gate(g, A, dt, lower_bound)
    if lower_bound is not None:
        assert (y < 0).all() and (y > lower_bound).all()
    else:
        assert (y < 0).all()
    dy = torch.randn(y.shape, generator=gen, dtype=torch.float64)
    want = torch.autograd.grad(y, [t for t in (g, A, dt) if t is not None], dy)
    got = [t for t in kda_gate_bwd(dy, g, A, dt, lower_bound) if t is not None]
    for a, b in zip(got, want):
        torch.testing.assert_close(a.double(), b, rtol=1e-5, atol=1e-6)


def test_public_kda_fused_gate_wiring_on_cpu():
    """chunk_kda(use_gate_in_kernel=True) == chunk_kda(g=activated gate), forward and
    gradients (original backend, CPU), including dA_log and ddt_bias."""
    import rewy_amd as fdr
    xs, dO = make_inputs("kda", 1, 128, 2, seed=3)
    gen = torch.Generator().manual_seed(9)
    g_raw = torch.randn(1, 128, 2, 128, generator=gen)
    A_log = torch.randn(2, generator=gen) * 0.5
    dt_bias = torch.randn(2 * 128, generator=gen) * 0.1
    leaves = dict(g=g_raw, A_log=A_log, dt_bias=dt_bias)
    a = {k: v.clone().requires_grad_() for k, v in leaves.items()}
    b = {k: v.clone().requires_grad_() for k, v in leaves.items()}
    with fdr.use_backend("original"):
        o1, _ = fdr.chunk_kda(xs["q"], xs["k"], xs["v"], a["g"], xs["beta"], initial_state=xs["initial_state"],
                              use_gate_in_kernel=True, A_log=a["A_log"], dt_bias=a["dt_bias"])
        g_act = -torch.exp(b["A_log"]).view(2, 1) * torch.nn.functional.softplus(b["g"] + b["dt_bias"].view(2, 128))
        o2, _ = fdr.chunk_kda(xs["q"], xs["k"], xs["v"], g_act, xs["beta"], initial_state=xs["initial_state"])
    torch.testing.assert_close(o1.float(), o2.float(), rtol=0, atol=0)
    g1 = torch.autograd.grad(o1, list(a.values()), dO)
    g2 = torch.autograd.grad(o2, list(b.values()), dO)
    for x, y in zip(g1, g2):
        torch.testing.assert_close(x, y, rtol=1e-5, atol=1e-6)
