"""The HIP KDA gate activation and its backward (fdr_kda_gate_fwd / _bwd) against the
torch expressions of the same documented activations (reference _compat/kda.py:250-294),
which tests/test_gates.py pins against fp64 autograd.  fp32 arithmetic both ways:
rel-L2 <= 1e-5 (the reductions dA_log / ddt_bias sum in another order)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _rel(a, r):
    a, r = a.double().cpu(), r.double().cpu()
    return float((a - r).norm() / r.norm().clamp_min(1e-30))


@pytest.mark.parametrize("mode", ["softplus", "bounded", "bounded_no_A"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_bias", [True, False])
@pytest.mark.parametrize("shape", [(2, 192, 3), (1, 448, 20)])
def test_hip_gate_matches_torch(mode, dtype, with_bias, shape):
    from rewy_amd.gates import kda_gate, kda_gate_bwd
    B, T, H = shape
    print(f"\n[gate] mode={mode} dtype={dtype} bias={with_bias} shape={shape}", flush=True)
    gen = torch.Generator().manual_seed(3)
    dev = torch.device("cuda")
    g_raw = (torch.randn(B, T, H, 128, generator=gen) * 3).to(dtype).to(dev)
    A = None if mode == "bounded_no_A" else (torch.randn(H, generator=gen) * 0.5).to(dev)
    dt = (torch.randn(H * 128, generator=gen) * 0.5).to(dev) if with_bias else None
    lb = None if mode == "softplus" else -5.0
    dg = torch.randn(B, T, H, 128, generator=gen).to(dev)
    got = kda_gate(g_raw, A, dt, lb, native=True)
    ref = kda_gate(g_raw, A, dt, lb, native=False)
    torch.cuda.synchronize()
    assert got.dtype == torch.float32 and _rel(got, ref) < 1e-6, _rel(got, ref)
    gb = kda_gate_bwd(dg, g_raw, A, dt, lb, native=True)
    rb = kda_gate_bwd(dg, g_raw, A, dt, lb, native=False)
    torch.cuda.synchronize()
    for name, a, r in zip(("dg_raw", "dA_log", "ddt_bias"), gb, rb):
        assert (a is None) == (r is None), name
        if r is None:
            continue
        assert a.dtype == r.dtype and a.shape == r.shape, name
        tol = 1e-5 if dtype == torch.float32 or name != "dg_raw" else 4e-3   # bf16 dg_raw: output rounding
        assert _rel(a, r) < tol, (name, _rel(a, r))
