"""Native variable-length batches: sequences packed along T on 64-token chunk boundaries,
the two state recurrences restarting at each sequence's first chunk
(fdr_state_bwd_varlen / fdr_fwd_h_varlen; the reference's state_bwd with cu_seqlens and
chunk_offsets, kernels/vector_state_gpu.py:47-67).

* ops level: the packed scans against the same kernels run on each sequence as its own
  batch row (same value-tile width, so the same arithmetic): bit-exact;
* public operators: packed cu_seqlens batches (lengths not multiples of 64, both saving
  policies) on the HIP path against the original backend at the reference's tolerances
  (rel-L2 0.008, 0.02 for gates)."""
import pytest
import torch

from oracle import delta_oracle as O
from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu

GATE = {"delta": 0, "gdn": 1, "kda": 2, "gdn2": 2}


@pytest.mark.parametrize("op", ["kda", "gdn", "delta"])
@pytest.mark.parametrize("vb", [16, 64])
def test_packed_scans_match_per_sequence_rows(op, vb):
    from rewy_amd import ops
    from rewy_amd.forward import chunk_forward
    lens, H = [64, 192, 128, 320], 3
    print(f"\n[varlen] scans op={op} lens={lens} H={H} vb={vb}", flush=True)
    T = sum(lens)
    xs, dO = make_inputs(op, 1, T, H, seed=21)
    _, _, sv = chunk_forward(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"))
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    vec = op == "kda"
    qs, ks = (sv["qg"], sv["kg"]) if vec else (xs["q"], xs["k"])
    q_, k_, w_, u_, g_, aqk, do = (cu(x) for x in (qs, ks, sv["w"], sv["u"], sv["gc"], sv["Aqk"], dO))
    gen = torch.Generator().manual_seed(8)
    N = len(lens)
    h0 = (torch.randn(N, H, 128, 128, generator=gen) * 0.1).to(dev)
    dht = (torch.randn(N, H, 128, 128, generator=gen) * 0.1).to(dev)
    offs = torch.tensor([0] + lens).cumsum(0)
    co = offs // 64
    gm = GATE[op]
    h, vn, ht = ops.fwd_h(k_, w_, u_, g_, gm, h0=h0, want_final=True, value_block=vb, chunk_offsets=co)
    dh, dR, dh0 = ops.state_bwd(q_, k_, w_, g_, gm, do, 1.0, aqk=aqk, dht=dht, value_block=vb, chunk_offsets=co)
    torch.cuda.synchronize()
    for n in range(N):
        a, e = int(offs[n]), int(offs[n + 1])
        ca, ce = a // 64, e // 64
        sl = lambda x: None if x is None else x[:, a:e].contiguous()
        rh, rvn, rht = ops.fwd_h(sl(k_), sl(w_), sl(u_), sl(g_), gm, h0=h0[n:n + 1].contiguous(), want_final=True,
                                 value_block=vb, method="direct")
        rdh, rdR, rdh0 = ops.state_bwd(sl(q_), sl(k_), sl(w_), sl(g_), gm, sl(do), 1.0, aqk=sl(aqk),
                                       dht=dht[n:n + 1].contiguous(), value_block=vb, method="direct")
        torch.cuda.synchronize()
        assert torch.equal(h[:, ca:ce], rh) and torch.equal(vn[:, a:e], rvn), n
        assert torch.equal(ht[n:n + 1], rht), n
        assert torch.equal(dh[:, ca:ce], rdh) and torch.equal(dR[:, a:e], rdR), n
        assert torch.equal(dh0[n:n + 1], rdh0), n


def test_chunk_offsets_are_validated():
    from rewy_amd import ops
    dev = torch.device("cuda")
    x = torch.zeros(1, 256, 1, 128, device=dev, dtype=torch.bfloat16)
    g = torch.zeros(1, 256, 1, 128, device=dev)
    for bad in ([0, 3], [1, 4], [0, 4, 3, 4], [0, 2, 1, 4]):
        with pytest.raises(ValueError, match="chunk_offsets"):
            ops.fwd_h(x, x, x, g, ops.GATE_VECTOR, chunk_offsets=torch.tensor(bad))
    with pytest.raises(ValueError, match="affine"):
        ops.fwd_h(x, x, x, g, ops.GATE_VECTOR, chunk_offsets=torch.tensor([0, 4]), method="affine")


def test_empty_sequences_pass_their_state_through():
    from rewy_amd import ops
    dev = torch.device("cuda")
    print("\n[varlen] empty sequences: offsets [0, 0, 2, 2, 4]", flush=True)
    gen = torch.Generator().manual_seed(5)
    r = lambda *s: (torch.randn(*s, generator=gen) * 0.1).to(dev)
    x = r(1, 256, 2, 128).bfloat16()
    g = -r(1, 256, 2, 128).abs()
    h0, dht = r(4, 2, 128, 128), r(4, 2, 128, 128)
    co = torch.tensor([0, 0, 2, 2, 4])
    _, _, ht = ops.fwd_h(x, x, x, g, ops.GATE_VECTOR, h0=h0, want_final=True, chunk_offsets=co)
    _, _, dh0 = ops.state_bwd(x, x, x, g, ops.GATE_VECTOR, x, 1.0, dv=x, dht=dht, chunk_offsets=co)
    torch.cuda.synchronize()
    for n in (0, 2):
        assert torch.equal(ht[n], h0[n]) and torch.equal(dh0[n], dht[n]), n
    assert not torch.equal(ht[1], h0[1]) and not torch.equal(dh0[3], dht[3])


@pytest.mark.parametrize("op,recompute,lens", [("kda", False, [1, 64, 300, 129, 700]),
                                               ("kda", True, [1, 64, 300, 129, 700]),
                                               ("gdn", True, [1, 64, 300, 129, 700]),
                                               ("gdn2", True, [1, 64, 300, 129, 700]),
                                               ("delta", True, [1, 64, 300, 129, 700]),
                                               ("kda", True, [128, 64, 576]),       # aligned: no repacking
                                               ("gdn", True, [64, 640])])
def test_packed_public_operators_match_original(op, recompute, lens):
    import rewy_amd as fdr
    from tests.test_gpu_e2e import OPNAME
    print(f"\n[varlen] e2e op={op} recompute={recompute} lens={lens}", flush=True)
    dev = torch.device("cuda")
    seqs = [make_inputs(op, 1, L, 2, seed=90 + i) for i, L in enumerate(lens)]
    names = list(seqs[0][0])
    packed = {n: torch.cat([x[n] for x, _ in seqs], 1 if n != "initial_state" else 0).to(dev) for n in names}
    dO = torch.cat([d for _, d in seqs], 1).to(dev)
    cu = torch.tensor([0] + lens).cumsum(0).to(dev)
    kw = dict(cu_seqlens=cu, output_final_state=True)
    if op in ("kda", "gdn2"):
        kw["disable_recompute"] = not recompute
    res = {}
    for backend in ("optimized", "original"):
        xg = {n: v.clone().requires_grad_() for n, v in packed.items()}
        with fdr.use_backend(backend, ops=(op,)):
            o, ht = getattr(fdr, OPNAME[op])(**xg, **kw)
        dht = (torch.randn(ht.shape, generator=torch.Generator().manual_seed(4)) * 0.1).to(dev)
        res[backend] = [o] + list(torch.autograd.grad((o, ht), list(xg.values()), (dO, dht))) + [ht]
    for name, a, r in zip(["o"] + names + ["final"], res["optimized"], res["original"]):
        lim = 0.02 if name in ("g", "beta", "b", "w") else 0.008
        e = O.error(r.detach().double().cpu().numpy(), a.detach().double().cpu().numpy(), lim)
        print(name, e, flush=True)
        assert e["passed"], (name, e)
