"""Layout adapters of the public operators (CPU, original backend): packed
variable-length batches (cu_seqlens), V-first states and grouped value heads,
each against the same computation written out by hand (separate sequences,
transposed states, repeated q/k heads) -- outputs, final states and gradients."""
import pytest
import torch

from tests._inputs import make_inputs

OPNAME = {"kda": "chunk_kda", "gdn": "chunk_gated_delta_rule", "gdn2": "chunk_gdn2", "delta": "chunk_delta_rule"}


def _call(op, xs, **kw):
    import rewy_amd as fdr
    extra = dict(disable_recompute=True) if op in ("kda", "gdn2") else {}
    with fdr.use_backend("original"):
        return getattr(fdr, OPNAME[op])(**xs, output_final_state=True, **extra, **kw)


@pytest.mark.parametrize("op", ["kda", "gdn", "gdn2", "delta"])
def test_varlen_equals_separate_sequences(op):
    lens = [100, 128, 37]
    seqs = [make_inputs(op, 1, L, 2, seed=40 + i) for i, L in enumerate(lens)]
    names = [n for n in seqs[0][0] if n != "initial_state"]
    packed = {n: torch.cat([x[n] for x, _ in seqs], 1).requires_grad_() for n in names}
    packed["initial_state"] = torch.cat([x["initial_state"] for x, _ in seqs], 0).requires_grad_()
    dO = torch.cat([d for _, d in seqs], 1)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()))
    o, ht = _call(op, packed, cu_seqlens=cu)
    dht = torch.randn(ht.shape, generator=torch.Generator().manual_seed(2)) * 0.1
    grads = torch.autograd.grad((o, ht), list(packed.values()), (dO, dht))
    start = 0
    for i, ((x, d), L) in enumerate(zip(seqs, lens)):
        xi = {n: v.clone().requires_grad_() for n, v in x.items()}
        oi, hi = _call(op, xi)
        torch.testing.assert_close(o[:, start:start + L].float(), oi.float(), rtol=2e-2, atol=2e-2)
        torch.testing.assert_close(ht[i:i + 1], hi, rtol=1e-4, atol=1e-4)
        gi = torch.autograd.grad((oi, hi), list(xi.values()), (d, dht[i:i + 1]))
        for n, gp, gs in zip(xi, grads, gi):
            sl = gp[i:i + 1] if n == "initial_state" else gp[:, start:start + L]
            torch.testing.assert_close(sl.float(), gs.float(), rtol=3e-2, atol=3e-2, msg=lambda m: f"{n}: {m}")
        start += L


@pytest.mark.parametrize("op", ["kda", "gdn", "gdn2"])
def test_state_v_first_is_the_transposed_state(op):
    xs, dO = make_inputs(op, 1, 128, 2, seed=50)
    a = {n: v.clone().requires_grad_() for n, v in xs.items()}
    b = {n: v.clone().requires_grad_() for n, v in xs.items()}
    b_in = dict(b, initial_state=b["initial_state"].transpose(-1, -2))
    o1, h1 = _call(op, a)
    o2, h2 = _call(op, b_in, state_v_first=True)
    torch.testing.assert_close(o1, o2, rtol=0, atol=0)
    torch.testing.assert_close(h1, h2.transpose(-1, -2), rtol=0, atol=0)
    dht = torch.randn(h1.shape, generator=torch.Generator().manual_seed(3))
    g1 = torch.autograd.grad((o1, h1), list(a.values()), (dO, dht))
    g2 = torch.autograd.grad((o2, h2), list(b.values()), (dO, dht.transpose(-1, -2)))
    for x, y in zip(g1, g2):
        torch.testing.assert_close(x, y, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("op", ["kda", "gdn"])
def test_grouped_value_heads(op):
    """HV = 4 value heads over H = 2 query/key heads == repeated q/k heads."""
    xs, dO = make_inputs(op, 1, 128, 4, seed=60)
    q2 = xs["q"][:, :, ::2].clone()
    k2 = xs["k"][:, :, ::2].clone()
    a = dict(xs, q=q2.clone().requires_grad_(), k=k2.clone().requires_grad_())
    o1, h1 = _call(op, a)
    b = dict(xs, q=q2.repeat_interleave(2, 2).requires_grad_(), k=k2.repeat_interleave(2, 2).requires_grad_())
    o2, h2 = _call(op, b)
    torch.testing.assert_close(o1, o2, rtol=0, atol=0)
    ga = torch.autograd.grad(o1, [a["q"], a["k"]], dO)
    gb = torch.autograd.grad(o2, [b["q"], b["k"]], dO)
    for x, y in zip(ga, gb):
        torch.testing.assert_close(x.float(), y.float().reshape(1, 128, 2, 2, 128).sum(3), rtol=1e-2, atol=1e-2)


def test_state_recurrence_form_routing():
    """Which form of the backward state recurrence the backend picks (host logic only):
    segmented for long rows with few heads, affine for few heads and few chunks, direct
    when B*H fills the GPU."""
    from rewy_amd import ops
    assert ops._state_method("auto", 1, 16, 1024) == "segmented"      # the long-context KDA config
    assert ops._state_method("auto", 8, 16, 64) == "direct"           # the headline config
    assert ops._state_method("auto", 2, 32, 128) == "direct"          # the GDN2 config
    assert ops._state_method("auto", 1, 4, 128) == "affine"           # the reference's grid, few chunks
    assert ops._state_method("auto", 1, 4, 17) == "affine"
    assert ops._state_method("auto", 1, 16, 16) == "direct"           # short rows: two launches fewer
    # segmented from fewer chunks below B*H = 32: 96 from B*H = 16, else 128 with B*H*NT >= 768
    assert ops._state_method("auto", 1, 16, 128) == "segmented"       # the grid's largest case
    assert ops._state_method("auto", 1, 24, 96) == "segmented" and ops._state_method("auto", 1, 24, 95) == "direct"
    assert ops._state_method("auto", 1, 16, 95) == "affine" and ops._state_method("auto", 1, 31, 96) == "segmented"
    assert ops._state_method("auto", 1, 32, 192) == "direct"
    # long rows: segmented below B*H = 48, direct from there
    assert ops._state_method("auto", 1, 32, 256) == "segmented" and ops._state_method("auto", 1, 47, 512) == "segmented"
    assert ops._state_method("auto", 1, 48, 256) == "direct" and ops._state_method("auto", 1, 96, 4096) == "direct"
    assert ops._state_method("auto", 1, 8, 128) == "segmented" and ops._state_method("auto", 1, 8, 127) == "affine"
    assert ops._state_method("auto", 1, 4, 192) == "segmented" and ops._state_method("auto", 1, 4, 191) == "affine"
    assert ops.segments_for(1, 16, 1024) == 8
    assert ops.segments_for(1, 1, 40) == 2                             # segments of >= 16 chunks
    assert ops._state_method("direct", 1, 16, 1024) == "direct"
