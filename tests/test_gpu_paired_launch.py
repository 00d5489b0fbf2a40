"""fdr_paired_recurrences (the state recurrence and the scan forming u in one launch) against
its two halves run as separate launches -- fdr_state_bwd / fdr_state_bwd_raw_qk and
fdr_fwd_h_u -- bit for bit: every family (the scalar / no-gate ones forming Aqk, or reading the
Aqk fdr_prepare_wu writes), value tiles 16 / 32 / 64, the vector gates with
prepared qg / kg / w and with raw q / k (w given or formed), grouped q / k heads, V-first
states, with and without the initial / final states; and the host-side argument rules."""
import pytest
import torch

from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu

GATE = {"kda": 2, "gdn2": 2, "gdn": 1, "delta": 0}


def _inputs(op, B, T, H, HQ, seed):
    from rewy_amd.forward import chunk_forward
    xs, _ = make_inputs(op, B, T, H, seed=seed)
    _, _, sv = chunk_forward(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"), b=xs.get("b"),
                             w=xs.get("w"), initial_state=xs["initial_state"])
    dev = torch.device("cuda")
    cu = lambda x: None if x is None else x.to(dev).contiguous()
    d = {n: cu(x) for n, x in xs.items()}
    d["Akk"], d["gc"], d["Aqk"] = cu(sv["Akk"]), cu(sv["gc"]), cu(sv.get("Aqk"))
    if HQ != H:
        d["q"], d["k"] = d["q"][:, :, ::H // HQ].contiguous(), d["k"][:, :, ::H // HQ].contiguous()
    gen = torch.Generator().manual_seed(seed + 1)
    d["dO"] = torch.randn(B, T, H, 128, generator=gen).to(dev, torch.bfloat16)
    d["dht"] = (torch.randn(B, H, 128, 128, generator=gen) * 0.1).to(dev)
    return d


def _check(got, ref, what):
    for n, a, r in zip(("dh", "dR", "dh0", "h", "v_new"), got[0] + got[1][:2], ref[0] + ref[1][:2]):
        if r is None:
            assert a is None, (what, n)
            continue
        assert torch.equal(a, r), (what, n, float((a.double() - r.double()).abs().max()))


@pytest.mark.parametrize("vb", [16, 32, 64])
@pytest.mark.parametrize("op,HQ", [("kda", 3), ("gdn2", 3), ("gdn", 3), ("delta", 3), ("kda", 1), ("gdn", 1)])
def test_one_launch_equals_the_two_launches(op, HQ, vb):
    from rewy_amd import ops
    B, T, H = 2, 320, 3
    print(f"\n[paired launch] op={op} HQ={HQ} value_block={vb}", flush=True)
    d = _inputs(op, B, T, H, HQ, 81)
    gate = GATE[op]
    vec = gate == 2
    gkw = dict(beta=d.get("beta"), w_gate=d.get("w"))
    pre = ops.prepare_wu(d["k"], d["v"], d["Akk"], gate, g=d["gc"], beta=d.get("beta"), b=d.get("b"), w=d.get("w"),
                         q=d["q"], want_qkg=vec, want_u=False)
    for vf in (False, True):
        for with_states in (True, False):
            h0 = d["initial_state"] if with_states and d.get("initial_state") is not None else None
            if h0 is not None and vf:
                h0 = h0.transpose(-1, -2).contiguous()
            dht = (d["dht"].transpose(-1, -2).contiguous() if vf else d["dht"]) if with_states else None
            st = dict(dht=dht, want_dh0=with_states, value_block=vb, method="direct", state_v_first=vf)
            sc = dict(h0=h0, value_block=vb, state_v_first=vf, **gkw)
            pk = dict(h0=h0, dht=dht, want_dh0=with_states, state_v_first=vf, **gkw)
            tag = (op, HQ, vb, vf, with_states)
            if not vec:
                ref = (ops.state_bwd(d["q"], d["k"], pre["w"], d["gc"], gate, d["dO"], 0.088, **st),
                       ops.fwd_h_u(d["k"], pre["w"], d["v"], d["Akk"], d["gc"], gate, **sc))
                got = ops.paired_recurrences(d["q"], d["k"], pre["w"], d["gc"], gate, d["dO"], 0.088, d["v"],
                                             d["Akk"], vb, **pk)
                torch.cuda.synchronize()
                _check(got, ref, tag)
                # Aqk written by prepare_wu (with or without u: the same w and Aqk) and read
                wa = ops.prepare_wu(d["k"], d["v"], d["Akk"], gate, g=d["gc"], beta=d["beta"], q=d["q"],
                                    want_aqk=True, scale=0.088, want_u=False)
                full = ops.prepare_wu(d["k"], d["v"], d["Akk"], gate, g=d["gc"], beta=d["beta"], q=d["q"],
                                      want_aqk=True, scale=0.088)
                torch.cuda.synchronize()
                assert torch.equal(wa["w"], pre["w"]) and torch.equal(wa["Aqk"], full["Aqk"]), tag
                ref = (ops.state_bwd(d["q"], d["k"], pre["w"], d["gc"], gate, d["dO"], 0.088, aqk=wa["Aqk"], **st),
                       ref[1])
                got = ops.paired_recurrences(d["q"], d["k"], pre["w"], d["gc"], gate, d["dO"], 0.088, d["v"],
                                             d["Akk"], vb, aqk=wa["Aqk"], **pk)
                torch.cuda.synchronize()
                _check(got, ref, tag + ("aqk read",))
                continue
            # qg / kg / w as prepare_wu wrote them
            ref = (ops.state_bwd(pre["qg"], pre["kg"], pre["w"], d["gc"], gate, d["dO"], 0.088, aqk=d["Aqk"], **st),
                   ops.fwd_h_u(d["k"], pre["w"], d["v"], d["Akk"], d["gc"], gate, kg=pre["kg"], **sc))
            got = ops.paired_recurrences(d["q"], d["k"], pre["w"], d["gc"], gate, d["dO"], 0.088, d["v"], d["Akk"],
                                         vb, aqk=d["Aqk"], qg=pre["qg"], kg=pre["kg"], **pk)
            torch.cuda.synchronize()
            _check(got, ref, tag + ("prepared",))
            if vb != 64:
                continue
            # raw q / k, w given
            ref = (ops.state_bwd(d["q"], d["k"], pre["w"], d["gc"], gate, d["dO"], 0.088, aqk=d["Aqk"],
                                 raw_qk=True, **st),
                   ops.fwd_h_u(d["k"], pre["w"], d["v"], d["Akk"], d["gc"], gate, **sc))
            got = ops.paired_recurrences(d["q"], d["k"], pre["w"], d["gc"], gate, d["dO"], 0.088, d["v"], d["Akk"],
                                         vb, aqk=d["Aqk"], raw_qk=True, **pk)
            torch.cuda.synchronize()
            _check(got, ref, tag + ("raw",))
            if op == "gdn2" and HQ != H:
                continue        # w formed from GDN2's b needs q / k heads = value heads
            # raw q / k, w formed in both
            ref = (ops.state_bwd(d["q"], d["k"], None, d["gc"], gate, d["dO"], 0.088, aqk=d["Aqk"], raw_qk=True,
                                 Akk=d["Akk"], beta=d.get("beta"), b=d.get("b"), **st),
                   ops.fwd_h_u(d["k"], None, d["v"], d["Akk"], d["gc"], gate, b=d.get("b"), **sc))
            got = ops.paired_recurrences(d["q"], d["k"], None, d["gc"], gate, d["dO"], 0.088, d["v"], d["Akk"], vb,
                                         aqk=d["Aqk"], raw_qk=True, b=d.get("b"), **pk)
            torch.cuda.synchronize()
            _check(got, ref, tag + ("w formed",))


def test_argument_rules():
    from rewy_amd import _lib, ops
    d = _inputs("kda", 1, 128, 2, 2, 82)
    pre = ops.prepare_wu(d["k"], d["v"], d["Akk"], 2, g=d["gc"], beta=d["beta"], q=d["q"], want_qkg=True,
                         want_u=False)
    base = dict(aqk=d["Aqk"], beta=d["beta"])
    with pytest.raises(ValueError):        # raw q / k only at 64-wide tiles
        ops.paired_recurrences(d["q"], d["k"], pre["w"], d["gc"], 2, d["dO"], 0.1, d["v"], d["Akk"], 32,
                               raw_qk=True, **base)
    with pytest.raises(ValueError):        # prepared qg / kg required without raw_qk
        ops.paired_recurrences(d["q"], d["k"], pre["w"], d["gc"], 2, d["dO"], 0.1, d["v"], d["Akk"], 32, **base)
    with pytest.raises(ValueError):        # the scalar families take the raw q / k only
        ops.paired_recurrences(d["q"], d["k"], pre["w"], d["gc"][..., 0].contiguous(), 1, d["dO"], 0.1, d["v"],
                               d["Akk"], 32, raw_qk=True, **base)
    # the library's own checks, below the Python ones
    P = _lib.ptr
    lib = _lib.load()
    x = d["q"]
    args = [P(x)] * 6 + [2] + [P(x)] * 15 + [0, 0, 1, 128, 2, 2, 128, 128, 64, 0.1, 48, None]
    assert lib.fdr_paired_recurrences(*args) != 0          # value_block 48
    args[-2] = 32
    args[22] = 1                                           # raw_qk at 32-wide tiles
    assert lib.fdr_paired_recurrences(*args) != 0


@pytest.mark.parametrize("vb", [16, 32, 64])
@pytest.mark.parametrize("op,HQ", [("gdn", 3), ("delta", 3), ("gdn", 1)])
def test_one_call_scalar_backward_equals_its_three_launches(op, HQ, vb):
    """fdr_scalar_bwd (ops.scalar_bwd) against fdr_prepare_wu, fdr_paired_recurrences and
    fdr_chunk_bwd called one by one, bit for bit: Aqk written by prepare or formed by the state
    recurrence, V-first states, with and without the initial / final states, beta_sigmoid."""
    from rewy_amd import ops
    B, T, H = 2, 320, 3
    print(f"\n[scalar one call] op={op} HQ={HQ} value_block={vb}", flush=True)
    d = _inputs(op, B, T, H, HQ, 83)
    gate = GATE[op]
    for aqk_pre in (False, True):
        for vf in (False, True):
            for with_states, sig in ((True, 0.0), (False, 2.0)):
                h0 = d["initial_state"] if with_states else None
                if h0 is not None and vf:
                    h0 = h0.transpose(-1, -2).contiguous()
                dht = (d["dht"].transpose(-1, -2).contiguous() if vf else d["dht"]) if with_states else None
                tag = (op, HQ, vb, aqk_pre, vf, with_states)
                pre = ops.prepare_wu(d["k"], d["v"], d["Akk"], gate, g=d["gc"], beta=d["beta"], q=d["q"],
                                     want_aqk=aqk_pre, scale=0.088, want_u=False)
                (dh, dr, dh0), (h, v_new, _) = ops.paired_recurrences(
                    d["q"], d["k"], pre["w"], d["gc"], gate, d["dO"], 0.088, d["v"], d["Akk"], vb, aqk=pre.get("Aqk"),
                    beta=d["beta"], h0=h0, dht=dht, want_dh0=with_states, state_v_first=vf)
                ref = ops.chunk_bwd(d["q"], d["k"], d["v"], v_new, d["dO"], dr, d["gc"], gate, d["Akk"], h, dh, 0.088,
                                    beta=d["beta"], beta_sigmoid=sig)
                got, gdh0 = ops.scalar_bwd(d["q"], d["k"], d["v"], d["gc"], gate, d["beta"], d["Akk"], d["dO"], 0.088,
                                           vb, aqk_pre, dht=dht, h0=h0, want_dh0=with_states, beta_sigmoid=sig,
                                           state_v_first=vf)
                torch.cuda.synchronize()
                for n in ("dq", "dk", "dv", "dg", "dbeta"):
                    if ref[n] is None:
                        assert got[n] is None, (tag, n)
                        continue
                    assert torch.equal(got[n], ref[n]), (tag, n, float((got[n].double() - ref[n].double()).abs().max()))
                assert (gdh0 is None) == (dh0 is None), tag
                if dh0 is not None:
                    assert torch.equal(gdh0, dh0), (tag, "dh0")
