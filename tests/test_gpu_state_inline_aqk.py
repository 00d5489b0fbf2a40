"""The reverse state recurrence forming Aqk itself (scalar / no gate: fdr_state_bwd with
neither aqk nor dv).  Aqk = scale tril(q k^T 2^(g_i - g_s)) is formed per chunk from the raw
q / k the recurrence stages (one bf16 tile, as FLA's chunk_bwd_dv_local rounds it), kg dh as
2^(g_last - g_t) (k dh) and qg^T dO as q^T (2^g dO):
against the fp64 oracle (its Aqk formed in fp64 from the same q, k, g) at the tolerances of
the stage tests (rel-L2 1e-2 for the bf16 dh / dR, 5e-3 for the fp32 dh0), for GDN and
DeltaNet, grouped q / k heads, every value-tile width and a packed batch whose sequences
start anywhere; and against the same recurrence reading the HIP forward's Aqk.
"""
import numpy as np
import pytest
import torch

from oracle import delta_oracle as O
from tests.test_gpu_stages import GATE, _np, _rel, _setup

pytestmark = pytest.mark.gpu


def _oracle_aqk(q, k, gc, scale, C=64):
    """scale tril(q k^T 2^(g_i - g_s)) per chunk, fp64 (rows [B,T,H,64])"""
    B, T, H, K = q.shape
    Q, Kc = O._to_chunks(q, C), O._to_chunks(k, C)
    G = O._to_chunks(np.zeros((B, T, H)) if gc is None else gc, C) if True else None
    s = scale * Q @ O._T(Kc)
    d = G[..., :, None] - G[..., None, :]
    low = np.tri(C, dtype=bool)
    s = np.where(low, s * np.exp2(np.where(low, d, 0.0)), 0.0)
    return O._from_chunks(s)


def _run(op, B, T, H, seed, vb, qk_groups=1):
    from rewy_amd import ops
    xs, dO, sv = _setup(op, B, T, H, seed=seed)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    scale = sv["scale"]
    q, k = xs["q"], xs["k"]
    if qk_groups > 1:
        q, k = q[:, :, ::qk_groups].contiguous(), k[:, :, ::qk_groups].contiguous()
    gc = sv["gc"]
    dht = torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(3)) * 0.1
    dh, dR, dh0 = ops.state_bwd(cu(q), cu(k), cu(sv["w"]), cu(gc), GATE[op], cu(dO), scale, dht=cu(dht),
                                value_block=vb, method="direct")
    torch.cuda.synchronize()
    qr = np.repeat(_np(q), qk_groups, axis=2)
    kr = np.repeat(_np(k), qk_groups, axis=2)
    gcn = np.zeros((B, T, H)) if gc is None else _np(gc)
    G = O._to_chunks(gcn[..., None], 64)
    oq = O._from_chunks(O._to_chunks(qr, 64) * np.exp2(G))
    ok_ = O._from_chunks(O._to_chunks(kr, 64) * np.exp2(G[..., -1:, :] - G))
    og = np.broadcast_to(gcn[..., None], (B, T, H, 128))
    odv = O.dv_local(_oracle_aqk(qr, kr, gcn, scale), _np(dO))
    rdh, rdR, rdh0 = O.stage_state_bwd(oq, ok_, _np(sv["w"]), og, _np(dO), odv, dht=_np(dht), scale=scale)
    e = dict(dh=_rel(_np(dh), rdh), dR=_rel(_np(dR), rdR), dh0=_rel(_np(dh0), rdh0))
    print(op, "inline-Aqk state vs oracle", e, flush=True)
    assert e["dh"] < 1e-2 and e["dR"] < 1e-2 and e["dh0"] < 5e-3, e
    return xs, dO, sv, (dh, dR, dh0)


@pytest.mark.parametrize("op", ["gdn", "delta"])
@pytest.mark.parametrize("vb", [16, 32, 64])
def test_inline_aqk_state_matches_the_oracle(op, vb):
    print(f"\n[inline-aqk] op={op} vb={vb}", flush=True)
    _run(op, 2, 256, 3, seed=41, vb=vb)


def test_inline_aqk_grouped_qk_heads():
    print("\n[inline-aqk] gdn grouped q/k heads", flush=True)
    _run("gdn", 1, 192, 4, seed=42, vb=0, qk_groups=2)


def test_inline_aqk_agrees_with_the_read_aqk():
    """the same recurrence reading the forward's Aqk instead: the two differ only in how
    Aqk and the gate factors are rounded"""
    from rewy_amd import ops
    print("\n[inline-aqk] vs read Aqk", flush=True)
    xs, dO, sv, got = _run("gdn", 2, 320, 2, seed=43, vb=0)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    dht = torch.randn(2, 2, 128, 128, generator=torch.Generator().manual_seed(3)) * 0.1
    ref = ops.state_bwd(cu(xs["q"]), cu(xs["k"]), cu(sv["w"]), cu(sv["gc"]), GATE["gdn"], cu(dO), sv["scale"],
                        aqk=cu(sv["Aqk"]), dht=cu(dht), method="direct")
    torch.cuda.synchronize()
    e = [_rel(_np(a), _np(b)) for a, b in zip(got, ref)]
    print("inline vs read", e, flush=True)
    assert max(e) < 5e-3, e


@pytest.mark.parametrize("op", ["gdn", "delta"])
def test_inline_aqk_packed_unaligned(op):
    """a packed batch whose sequences start anywhere: the in-kernel Aqk of masked partial
    chunks equals the padded layout's (the seam path, against the padded-chunk run)"""
    from tests.test_gpu_varlen_unaligned import _pad, _run as run_seam, _unpad, LENS
    from tests._inputs import make_inputs
    print(f"\n[inline-aqk] packed op={op}", flush=True)
    lens, H = LENS, 2
    T = sum(lens)
    dev = torch.device("cuda")
    xs, dO = make_inputs(op, 1, T, H, seed=44)
    gen = torch.Generator().manual_seed(45)
    xs["initial_state"] = torch.randn(len(lens), H, 128, 128, generator=gen) * 0.05
    dht = (torch.randn(len(lens), H, 128, 128, generator=gen) * 0.05).to(dev)
    xs = {n: x.to(dev) for n, x in xs.items()}
    cu = torch.tensor([0] + lens).cumsum(0)
    cu_p = torch.tensor([0] + [-(-L // 64) * 64 for L in lens]).cumsum(0)
    padded = {n: (x if n == "initial_state" else _pad(x, lens)) for n, x in xs.items()}
    _, _, _, gr = run_seam(op, xs, dO.to(dev), dht, cu.to(dev), "recompute")
    _, _, _, pgr = run_seam(op, padded, _pad(dO.to(dev), lens), dht, cu_p.to(dev), "recompute")
    # DeltaNet: bit for bit.  GDN: the chunk's g_last (read at the last row that exists, vs the
    # padded layout's scan value at row 63, equal but for the last bit) enters dR as the fp32
    # row factor 2^(g_last - g_t) before dR is rounded to bf16, so a few roundings flip
    tol = 0.0 if op == "delta" else 1e-4
    for n, a in gr.items():
        if a is None:
            continue
        b = pgr[n] if n == "dh0" else _unpad(pgr[n], lens)
        e = float((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-30))
        print(n, e, flush=True)
        assert e <= tol, (n, e)


@pytest.mark.parametrize("op", ["gdn", "delta"])
@pytest.mark.parametrize("vb", [16, 32, 64])
def test_inline_aqk_packed_every_tile_width(op, vb):
    """The in-kernel-Aqk recurrence on a packed batch whose sequences start anywhere, at every
    value-tile width (64-wide tiles form each chunk's Aqk one step ahead): against the same
    batch zero-padded to whole chunks on the dense kernel with chunk offsets.  DeltaNet bit for
    bit; GDN within rel-L2 1e-4 (g_last, as above)."""
    from rewy_amd import ops
    from tests.test_gpu_varlen_unaligned import LENS, _pad, _unpad
    print(f"\n[inline-aqk] packed every tile width op={op} vb={vb}", flush=True)
    lens, H = LENS, 2
    T = sum(lens)
    dev = torch.device("cuda")
    gen = torch.Generator().manual_seed(46)
    bf = torch.bfloat16
    q = torch.nn.functional.normalize(torch.randn(1, T, H, 128, generator=gen), dim=-1).to(bf)
    k = torch.nn.functional.normalize(torch.randn(1, T, H, 128, generator=gen), dim=-1).to(bf)
    w = (torch.randn(1, T, H, 128, generator=gen) * 0.1).to(bf)
    dO = torch.randn(1, T, H, 128, generator=gen).to(bf)
    dht = torch.randn(len(lens), H, 128, 128, generator=gen) * 0.05
    g = None
    if op == "gdn":
        # chunk-local cumsum (log2) of each sequence's decays, the padded rows adding zero
        inc = torch.nn.functional.logsigmoid(torch.randn(1, T, H, generator=gen) * 0.5 + 4)
        inc_p = _pad(inc, lens)
        g_p = inc_p.view(1, -1, 64, H).cumsum(2).view(1, -1, H) / 0.6931471805599453
        g = _unpad(g_p, lens).contiguous()
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    gate = GATE[op]
    vl = ops.Varlen(torch.tensor([0] + lens).cumsum(0), dev)
    vl_p = ops.Varlen(torch.tensor([0] + [-(-L // 64) * 64 for L in lens]).cumsum(0), dev)
    got = ops.state_bwd(cu(q), cu(k), cu(w), cu(g), gate, cu(dO), 0.088, dht=cu(dht), value_block=vb,
                        method="direct", varlen=vl)
    P = lambda x: None if x is None else cu(_pad(x, lens))
    ref = ops.state_bwd(P(q), P(k), P(w), None if g is None else cu(g_p), gate, P(dO), 0.088, dht=cu(dht),
                        value_block=vb, method="direct", varlen=vl_p)
    torch.cuda.synchronize()
    tol = 0.0 if op == "delta" else 1e-4
    for n, a, b in (("dh", got[0], ref[0]), ("dR", got[1], _unpad(ref[1], lens)), ("dh0", got[2], ref[2])):
        e = float((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-30))
        print(n, e, flush=True)
        assert e <= tol, (n, e)
