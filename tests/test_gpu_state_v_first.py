"""V-first states (FLA's ``state_v_first``: [.., V, K] instead of [.., K, V]) read and
written by the kernels themselves (reference _compat/kda.py:485-493,
kernels/vector_state_gpu.py:24-25).

The V-first path only changes where each element is read or written, so every result
must equal the K-first run on transposed inputs bit for bit: the state recurrences
(direct, variable length, segmented, affine-step), the forward scan (direct, variable
length, affine-step), the chunk kernel reading a V-first saved h (plain and with the
folded gate), and the backward seam kda_backward / gdn2_backward against their K-first
runs on the same values.
"""
import pytest
import torch

from tests.test_gpu_stages import GATE, _setup

pytestmark = pytest.mark.gpu


def _t(x):
    return None if x is None else x.transpose(-1, -2).contiguous()


def _eq(a, b, name):
    assert a.shape == b.shape, name
    assert torch.equal(a, b), (name, float((a.float() - b.float()).abs().max()))


@pytest.mark.parametrize("op,shape,method", [("kda", (2, 64 * 5, 2), "direct"), ("gdn", (1, 64 * 12, 2), "affine"),
                                             ("gdn2", (1, 64 * 20, 1), "segmented"), ("delta", (2, 64 * 3, 3), "direct")])
def test_state_recurrences_v_first(op, shape, method):
    from rewy_amd import ops
    B, T, H = shape
    print(f"\n[v-first] state op={op} shape={shape} method={method}", flush=True)
    xs, dO, sv = _setup(op, B, T, H, seed=51)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    vec = op in ("kda", "gdn2")
    qs, ks = (sv["qg"], sv["kg"]) if vec else (xs["q"], xs["k"])
    dht = torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(2)).to(dev) * 0.1
    args = (cu(qs), cu(ks), cu(sv["w"]), cu(sv["gc"]), GATE[op], cu(dO), sv["scale"])
    kw = dict(aqk=cu(sv["Aqk"]), method=method, segments=4 if method == "segmented" else 0)
    dh, dR, dh0 = ops.state_bwd(*args, dht=dht, **kw)
    vdh, vdR, vdh0 = ops.state_bwd(*args, dht=_t(dht), state_v_first=True, **kw)
    h0 = cu(xs.get("initial_state"))
    fk = (cu(ks), cu(sv["w"]), cu(sv["u"]), cu(sv["gc"]), GATE[op])
    fmethod = "affine" if method == "affine" else "direct"
    h, vn, ht = ops.fwd_h(*fk, h0=h0, want_final=True, method=fmethod)
    vh, vvn, vht = ops.fwd_h(*fk, h0=_t(h0), want_final=True, method=fmethod, state_v_first=True)
    torch.cuda.synchronize()
    _eq(vdh, dh, "dh")
    _eq(vdR, dR, "dR")
    _eq(vdh0, _t(dh0), "dh0")
    _eq(vh, h, "h")
    _eq(vvn, vn, "v_new")
    _eq(vht, _t(ht), "final")


def test_varlen_scans_v_first():
    from rewy_amd import ops
    print("\n[v-first] varlen scans", flush=True)
    xs, dO, sv = _setup("kda", 1, 64 * 6, 2, seed=52)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    co = torch.tensor([0, 2, 2, 6], dtype=torch.int32, device=dev)       # an empty sequence in the middle
    dht = torch.randn(3, 2, 128, 128, generator=torch.Generator().manual_seed(3)).to(dev) * 0.1
    args = (cu(sv["qg"]), cu(sv["kg"]), cu(sv["w"]), cu(sv["gc"]), 2, cu(dO), sv["scale"])
    dh, dR, dh0 = ops.state_bwd(*args, aqk=cu(sv["Aqk"]), dht=dht, chunk_offsets=co)
    vdh, vdR, vdh0 = ops.state_bwd(*args, aqk=cu(sv["Aqk"]), dht=_t(dht), chunk_offsets=co, state_v_first=True)
    fk = (cu(sv["kg"]), cu(sv["w"]), cu(sv["u"]), cu(sv["gc"]), 2)
    h, vn, ht = ops.fwd_h(*fk, h0=dht, want_final=True, chunk_offsets=co)
    vh, vvn, vht = ops.fwd_h(*fk, h0=_t(dht), want_final=True, chunk_offsets=co, state_v_first=True)
    torch.cuda.synchronize()
    for n, a, b in (("dh", vdh, dh), ("dR", vdR, dR), ("dh0", vdh0, _t(dh0)), ("h", vh, h), ("v_new", vvn, vn),
                    ("final", vht, _t(ht))):
        _eq(a, b, n)


@pytest.mark.parametrize("op,fold", [("kda", False), ("kda", True), ("gdn2", False)])
def test_chunk_kernel_reads_v_first_saved_states(op, fold):
    from rewy_amd import ops
    print(f"\n[v-first] chunk kernel op={op} fold={fold}", flush=True)
    B, T, H = 2, 192, 3
    xs, dO, sv = _setup(op, B, T, H, seed=53)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    dh, dR, _ = ops.state_bwd(cu(sv["qg"]), cu(sv["kg"]), cu(sv["w"]), cu(sv["gc"]), 2, cu(dO), sv["scale"],
                              aqk=cu(sv["Aqk"]))
    kw = dict(beta=cu(xs.get("beta")), b=cu(xs.get("b")), w=cu(xs.get("w")))
    if fold:
        gen = torch.Generator().manual_seed(4)
        kw["gate_fold"] = dict(g_raw=torch.randn(B, T, H, 128, generator=gen).to(dev),
                               A_log=(torch.randn(H, generator=gen) * 0.5).to(dev), dt_bias=None, lower_bound=None)
    args = (cu(xs["q"]), cu(xs["k"]), cu(xs["v"]), cu(sv["v_new"]), cu(dO), dR, cu(sv["gc"]), 2, cu(sv["Akk"]))
    ref = ops.chunk_bwd(*args, cu(sv["h"]), dh, sv["scale"], **kw)
    got = ops.chunk_bwd(*args, _t(cu(sv["h"])), dh, sv["scale"], h_v_first=True, **kw)
    torch.cuda.synchronize()
    for name, r in ref.items():
        if r is not None:
            _eq(got[name], r, name)


@pytest.mark.parametrize("op,saving", [("kda", "full"), ("kda", "recompute"), ("gdn2", "full")])
def test_backward_seam_v_first(op, saving):
    """kda_backward / gdn2_backward(state_v_first=True) with V-first initial_state, dht and
    (full saving) saved h, against the K-first call on the same values."""
    from rewy_amd.backends import backward as bw
    print(f"\n[v-first] seam op={op} saving={saving}", flush=True)
    B, T, H = 1, 256, 2
    xs, dO, sv = _setup(op, B, T, H, seed=54)
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    h0 = cu(xs["initial_state"])
    dht = torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(5)).to(dev) * 0.1
    full = saving == "full"
    saved = {n: (cu(sv[n]) if full else None) for n in ("w", "u", "qg", "kg", "v_new", "h")}
    common = dict(q=cu(xs["q"]), k=cu(xs["k"]), v=cu(xs["v"]), Aqk=cu(sv["Aqk"]), Akk=cu(sv["Akk"]),
                  scale=sv["scale"], do=cu(dO), g=cu(sv["gc"]))
    if op == "kda":
        call = lambda vf, h0_, dht_, h_: bw.kda_backward(beta=cu(xs["beta"]), initial_state=h0_, dht=dht_,
                                                         state_v_first=vf, **common, **dict(saved, h=h_))
    else:
        call = lambda vf, h0_, dht_, h_: bw.gdn2_backward(b=cu(xs["b"]), w_gate=cu(xs["w"]), initial_state=h0_,
                                                          dht=dht_, state_v_first=vf, w_wy=saved["w"],
                                                          u_wy=saved["u"], qg=saved["qg"], kg=saved["kg"],
                                                          v_new=saved["v_new"], h=h_, **common)
    ref = call(False, h0, dht, saved["h"])
    got = call(True, _t(h0), _t(dht), _t(saved["h"]) if full else None)
    torch.cuda.synchronize()
    dh0_index = 5 if op == "kda" else 6
    for i, (a, r) in enumerate(zip(got, ref)):
        if r is None:
            assert a is None
            continue
        _eq(a, _t(r) if i == dh0_index else r, f"output {i}")
