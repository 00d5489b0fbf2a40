"""Packed variable-length batches whose sequences start anywhere, taken by the kernels
themselves (FLA's IS_VARLEN indexing that the reference's kernels use,
kernels/endpoint_intra.py:58-63: cu_seqlens, chunk_indices, chunk_offsets; each sequence
cut into ceil(len / 64) chunks, the last one partial).

The masked rows of a partial chunk (zero data rows, gate cumsum rows held at the last row
that exists, no stores) restate exactly the arithmetic of the sequence zero-padded to whole
chunks.  So every result of the packed run must equal, bit for bit, the same batch
zero-padded to whole chunks and run on the dense kernels with chunk offsets (the layout the
scans take and the public operators used to build by copies): forward outputs and final
states, the saved per-chunk states, and every gradient of the backward seams, for the four
families and both saving policies.  One exception, GDN's scalar gate: the chunk's decay
is 2^(g at its last row), which the packed run reads at the last row that exists (FLA's
g_last) while the padded run reads the cumsum scan's value at row 63, equal in exact
arithmetic (the pad adds zeros) but summed in another order, a last-bit difference that
reaches the final states, dh0 and dg (held to rel-L2 1e-6 there).  The lengths hold partial chunks, a one-token sequence
and an empty one (which owns no chunk and passes its state through).  The public operators
on such batches are checked against the original backend in test_gpu_varlen.py.
"""
import pytest
import torch

from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu

LENS = [100, 37, 0, 64, 1, 150]
GATE = {"delta": 0, "gdn": 1, "kda": 2, "gdn2": 2}


def _pad(x, lens):
    """packed [1, T, ...] -> [1, Tp, ...], each sequence zero-padded to whole chunks"""
    out, a = [], 0
    for L in lens:
        Lp = -(-L // 64) * 64
        seq = x[:, a:a + L]
        out.append(torch.nn.functional.pad(seq, [0, 0] * (x.ndim - 2) + [0, Lp - L]))
        a += L
    return torch.cat(out, 1).contiguous()


def _unpad(x, lens):
    out, a = [], 0
    for L in lens:
        out.append(x[:, a:a + L])
        a += -(-L // 64) * 64
    return torch.cat(out, 1)


def _eq(a, b, name, rel=0.0):
    assert a.shape == b.shape, (name, a.shape, b.shape)
    if rel:
        e = float((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-30))
        assert e <= rel, (name, e)
        return
    assert torch.equal(a, b), (name, float((a.float() - b.float()).abs().max()))


def _run(op, xs, dO, dht, cu, saving):
    """HIP forward (chunk_forward_hip) and the backward seam on one packed batch."""
    from rewy_amd import ops
    from rewy_amd.backends import backward as bw
    from rewy_amd.hip_forward import chunk_forward_hip
    dev = dO.device
    vl = ops.Varlen(cu, dev)
    o, final, sv = chunk_forward_hip(op, xs["q"], xs["k"], xs["v"], g=xs.get("g"), beta=xs.get("beta"),
                                     b=xs.get("b"), w=xs.get("w"), initial_state=xs["initial_state"],
                                     output_final_state=True, varlen=vl)
    scale = sv["scale"]
    full = saving == "full"
    common = dict(q=xs["q"], k=xs["k"], v=xs["v"], scale=scale, initial_state=xs["initial_state"], do=dO, dht=dht,
                  cu_seqlens=cu)
    if op == "kda":
        kept = {n: (sv[n] if full else None) for n in ("w", "u", "qg", "kg", "v_new", "h")}
        grads = bw.kda_backward(beta=xs["beta"], Aqk=sv["Aqk"], Akk=sv["Akk"], g=sv["gc"], **kept, **common)[:6]
        names = ("dq", "dk", "dv", "dbeta", "dg", "dh0")
    elif op == "gdn2":
        kept = dict(w_wy=sv["w"], u_wy=sv["u"], qg=sv["qg"], kg=sv["kg"], v_new=sv["v_new"], h=sv["h"]) if full else {}
        grads = bw.gdn2_backward(b=xs["b"], w_gate=xs["w"], Aqk=sv["Aqk"], Akk=sv["Akk"], g=sv["gc"], **kept,
                                 **common)[:7]
        names = ("dq", "dk", "dv", "db", "dw", "dg", "dh0")
    elif op == "gdn":
        grads = bw.gdn_backward(g=sv["gc"], beta=xs["beta"], A=sv["Akk"], **common)[:6]
        names = ("dq", "dk", "dv", "dbeta", "dg", "dh0")
    else:
        grads = bw.delta_backward(beta=xs["beta"], A=sv["Akk"], **common)
        names = ("dq", "dk", "dv", "dbeta", "dh0")
    torch.cuda.synchronize()
    return o, final, sv, dict(zip(names, grads))


@pytest.mark.parametrize("op,saving", [("kda", "full"), ("kda", "recompute"), ("gdn2", "full"),
                                       ("gdn2", "recompute"), ("gdn", "recompute"), ("delta", "recompute")])
def test_unaligned_packed_batch_equals_padded_chunks(op, saving):
    lens, H = LENS, 2
    T = sum(lens)
    print(f"\n[varlen-unaligned] op={op} saving={saving} lens={lens} H={H}", flush=True)
    dev = torch.device("cuda")
    xs, dO = make_inputs(op, 1, T, H, seed=71)
    N = len(lens)
    gen = torch.Generator().manual_seed(72)
    xs["initial_state"] = torch.randn(N, H, 128, 128, generator=gen) * 0.05
    dht = (torch.randn(N, H, 128, 128, generator=gen) * 0.05).to(dev)
    xs = {n: x.to(dev) for n, x in xs.items()}
    dO = dO.to(dev)
    cu = torch.tensor([0] + lens).cumsum(0)
    cu_p = torch.tensor([0] + [-(-L // 64) * 64 for L in lens]).cumsum(0)
    padded = {n: (x if n == "initial_state" else _pad(x, lens)) for n, x in xs.items()}
    o, final, sv, gr = _run(op, xs, dO, dht, cu.to(dev), saving)
    po, pfinal, psv, pgr = _run(op, padded, _pad(dO, lens), dht, cu_p.to(dev), saving)
    rel = 1e-6 if op == "gdn" else 0.0           # the scalar gate's g_last (see above)
    _eq(o, _unpad(po, lens), "o")
    _eq(final, pfinal, "final", rel)
    for n in ("gc", "Aqk", "Akk", "w", "u", "qg", "kg", "v_new"):
        if sv.get(n) is not None:
            _eq(sv[n], _unpad(psv[n], lens), n)
    _eq(sv["h"], psv["h"], "h")                  # per chunk: the same chunk list
    for n, a in gr.items():
        if a is None:
            assert pgr[n] is None, n
            continue
        _eq(a, pgr[n] if n == "dh0" else _unpad(pgr[n], lens), n, rel if n in ("dh0", "dg") else 0.0)


def _rel(a, r):
    a, r = a.double().cpu(), r.double().cpu()
    return float((a - r).norm() / r.norm().clamp_min(1e-30))


@pytest.mark.parametrize("mode", ["softplus", "bounded", "bounded_no_A"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_unaligned_seam_with_the_kda_gate(mode, dtype):
    """kda_backward(use_gate_in_kernel=True) on a batch whose sequences start anywhere (a
    partial chunk, a one-token and an empty sequence): the gate's backward is folded into
    the chunk kernel (fdr_chunk_bwd_gate_fold_varlen), rows past a sequence's end adding
    nothing to dA_log / ddt_bias.  Its dg_raw, dA_log and ddt_bias against the torch
    restatement of the gate backward applied to the same call's dg without the gate (rel-L2
    1e-5; dg_raw 4e-3 when stored in bf16); the other gradients equal that call's."""
    from rewy_amd import gates, ops
    from rewy_amd.backends import backward as bw
    from rewy_amd.hip_forward import chunk_forward_hip
    lens, H = [70, 3, 0, 190, 1], 2
    T = sum(lens)
    print(f"\n[varlen-unaligned] kda gate lens={lens} mode={mode} dtype={dtype}", flush=True)
    dev = torch.device("cuda")
    xs, dO = make_inputs("kda", 1, T, H, seed=73)
    gen = torch.Generator().manual_seed(74)
    g_raw = (torch.randn(1, T, H, 128, generator=gen) * 3).to(dtype).to(dev)
    A_log = None if mode == "bounded_no_A" else (torch.randn(H, generator=gen) * 0.5).to(dev)
    dt_bias = (torch.randn(H * 128, generator=gen) * 0.5).to(dev)
    lb = None if mode == "softplus" else -5.0
    x = {n: v.to(dev) for n, v in xs.items() if n != "initial_state"}
    dO = dO.to(dev)
    cu = torch.tensor([0] + lens).cumsum(0).to(dev)
    g = gates.kda_gate(g_raw, A_log, dt_bias, lb, native=True)
    _, _, sv = chunk_forward_hip("kda", x["q"], x["k"], x["v"], g=g, beta=x["beta"], varlen=ops.Varlen(cu, dev))
    kw = dict(q=x["q"], k=x["k"], v=x["v"], beta=x["beta"], Aqk=sv["Aqk"], Akk=sv["Akk"], scale=sv["scale"],
              initial_state=None, do=dO, dht=None, g=sv["gc"], cu_seqlens=cu)
    got = bw.kda_backward(**kw, g_org=g_raw, use_gate_in_kernel=True, A_log=A_log, dt_bias=dt_bias, lower_bound=lb)
    plain = bw.kda_backward(**kw)
    torch.cuda.synchronize()
    for i, n in enumerate(("dq", "dk", "dv", "dbeta")):
        _eq(got[i], plain[i], n)
    assert got[4].dtype == dtype
    dx, dA, ddt = gates.kda_gate_bwd(plain[4], g_raw, A_log, dt_bias, lb, native=False)
    assert _rel(got[4], dx) < (1e-5 if dtype == torch.float32 else 4e-3), _rel(got[4], dx)
    assert (got[6] is None) == (dA is None)
    if dA is not None:
        assert _rel(got[6], dA) < 1e-5, _rel(got[6], dA)
    assert _rel(got[7], ddt) < 1e-5, _rel(got[7], ddt)
