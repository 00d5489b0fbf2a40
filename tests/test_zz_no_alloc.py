"""fdr_chunk_bwd_gate_fold_noalloc (no workspace argument: the per-chunk partials sit in
the library's fixed device array) against fdr_chunk_bwd_gate_fold with a caller-allocated
workspace, through the C-ABI.  Both launch the same kernels, so every output must be
bit-identical; two calls in a row, the second on a smaller problem (the array keeps the
first call's partials, which the second must not read), then a size beyond the array's
limit is refused.  Also with V-first saved states (h_v_first = 1), and captured in a HIP
graph after one eager call (the per-device set-up happens on that call): three replays, with
eager work between them, each bit-identical to the workspace entry point."""
import pytest
import torch

from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu

HIP_ERROR_INVALID_VALUE = 1


def _lib():
    from rewy_amd import _lib as L
    return L, L.load()


def _case(B, T, H, seed):
    from rewy_amd import ops
    from rewy_amd.forward import chunk_forward
    xs, dO = make_inputs("kda", B, T, H, seed=seed)
    _, _, sv = chunk_forward("kda", xs["q"], xs["k"], xs["v"], g=xs["g"], beta=xs["beta"],
                             initial_state=xs["initial_state"])
    dev = torch.device("cuda")
    cu = lambda x: x.to(dev).contiguous()
    gen = torch.Generator().manual_seed(seed + 1)
    g_raw = (torch.randn(B, T, H, 128, generator=gen) * 3).to(dev)
    A = (torch.randn(H, generator=gen) * 0.5).to(dev)
    dt = (torch.randn(H * 128, generator=gen) * 0.5).to(dev)
    gc = cu(sv["gc"])
    dh, dR, _ = ops.state_bwd(cu(sv["qg"]), cu(sv["kg"]), cu(sv["w"]), gc, ops.GATE_VECTOR, cu(dO), sv["scale"],
                              aqk=cu(sv["Aqk"]))
    ins = [cu(xs["q"]), cu(xs["k"]), cu(xs["v"]), cu(sv["v_new"]), cu(dO), dR, gc, cu(xs["beta"]), cu(sv["Akk"]),
           cu(sv["h"]), dh]
    return ins, g_raw, A, dt, sv["scale"]


def _outs(B, T, H, dev):
    e = lambda *s: torch.full(s, float("nan"), device=dev)
    return dict(dq=e(B, T, H, 128).bfloat16(), dk=e(B, T, H, 128).bfloat16(), dv=e(B, T, H, 128).bfloat16(),
                dbeta=e(B, T, H), dg=e(B, T, H, 128), dA=e(H), ddt=e(H * 128))


def _call(L, lib, ins, g_raw, A, dt, scale, shape, noalloc, hvf=0, out=None, sync=True):
    B, T, H = shape
    dev = g_raw.device
    out = _outs(B, T, H, dev) if out is None else out
    P = L.ptr
    head = [P(x) for x in ins] + [P(out["dq"]), P(out["dk"]), P(out["dv"]), P(out["dbeta"]), 0.0, P(g_raw), 0,
                                  P(A), P(dt), 0, 0.0, P(out["dg"]), P(out["dA"]), P(out["ddt"])]
    tail = [hvf, B, T, H, 0, 128, 128, 64, float(scale), L.stream_handle(dev)]
    if noalloc:
        st = lib.fdr_chunk_bwd_gate_fold_noalloc(*head, *tail)
    else:
        ws = torch.empty(lib.fdr_chunk_bwd_gate_workspace_bytes(B, T, H) // 4, device=dev)
        st = lib.fdr_chunk_bwd_gate_fold(*head, P(ws), *tail)
    if sync:
        torch.cuda.synchronize()
    return st, out


def test_noalloc_matches_workspace_entry_point():
    L, lib = _lib()
    for shape, seed in (((2, 256, 4), 3), ((1, 128, 2), 8)):
        print(f"\n[no-alloc] shape={shape} seed={seed}", flush=True)
        ins, g_raw, A, dt, scale = _case(*shape, seed)
        st_ref, ref = _call(L, lib, ins, g_raw, A, dt, scale, shape, noalloc=False)
        st_got, got = _call(L, lib, ins, g_raw, A, dt, scale, shape, noalloc=True)
        assert st_ref == 0 and st_got == 0, (st_ref, st_got)
        for name in ref:
            assert torch.isfinite(got[name].float()).all(), name
            assert torch.equal(got[name], ref[name]), name


def test_noalloc_rejects_sizes_beyond_its_array():
    L, lib = _lib()
    dev = torch.device("cuda")
    # B * T/64 * (H*128 + 8 H) * 4 bytes = 35.7 MB > 16 MiB for B=16, T=16384, H=16
    B, T, H = 16, 16384, 16
    assert lib.fdr_chunk_bwd_gate_workspace_bytes(B, T, H) > (16 << 20)
    dummy = torch.empty(16, device=dev)
    p = L.ptr(dummy)
    st = lib.fdr_chunk_bwd_gate_fold_noalloc(*([p] * 15), 0.0, p, 0, p, None, 0, 0.0, p, p, None, 0,
                                             B, T, H, 0, 128, 128, 64, 1.0, L.stream_handle(dev))
    assert st == HIP_ERROR_INVALID_VALUE


def test_noalloc_with_v_first_states():
    L, lib = _lib()
    shape = (1, 192, 3)
    print(f"\n[no-alloc] h_v_first shape={shape}", flush=True)
    ins, g_raw, A, dt, scale = _case(*shape, 11)
    ins[9] = ins[9].transpose(-1, -2).contiguous()          # saved h as [B,NT,H,V,K]
    st_ref, ref = _call(L, lib, ins, g_raw, A, dt, scale, shape, noalloc=False, hvf=1)
    st_got, got = _call(L, lib, ins, g_raw, A, dt, scale, shape, noalloc=True, hvf=1)
    assert st_ref == 0 and st_got == 0, (st_ref, st_got)
    for name in ref:
        assert torch.equal(got[name], ref[name]), name


def test_noalloc_under_graph_capture():
    L, lib = _lib()
    shape = (2, 128, 2)
    print(f"\n[no-alloc] graph capture shape={shape}", flush=True)
    ins, g_raw, A, dt, scale = _case(*shape, 12)
    st_ref, ref = _call(L, lib, ins, g_raw, A, dt, scale, shape, noalloc=False)
    assert st_ref == 0
    st, _ = _call(L, lib, ins, g_raw, A, dt, scale, shape, noalloc=True)      # eager first call
    assert st == 0
    out = _outs(*shape, g_raw.device)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            # the library launches on the stream it is given: the capturing one
            st, _ = _call(L, lib, ins, g_raw, A, dt, scale, shape, noalloc=True, out=out, sync=False)
    torch.cuda.current_stream().wait_stream(side)
    assert st == 0
    for rep in range(3):
        for x in out.values():
            x.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for name in ref:
            assert torch.equal(out[name], ref[name]), (rep, name)
        st, _ = _call(L, lib, ins, g_raw, A, dt, scale, (1, 128, 2), noalloc=True)   # eager work between
        assert st == 0


_FIRST_CALL_CAPTURED = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
from tests.test_zz_no_alloc import _case, _call, _outs, _lib
L, lib = _lib()
shape = (1, 128, 2)
ins, g_raw, A, dt, scale = _case(*shape, 13)
torch.cuda.synchronize()
out = _outs(*shape, g_raw.device)
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(side):
    with torch.cuda.graph(graph, stream=side):
        # the entry point's first call in this process: its per-device set-up runs under capture
        st, _ = _call(L, lib, ins, g_raw, A, dt, scale, shape, noalloc=True, out=out, sync=False)
torch.cuda.current_stream().wait_stream(side)
assert st == 0, st
st_ref, ref = _call(L, lib, ins, g_raw, A, dt, scale, shape, noalloc=False)   # after the capture
assert st_ref == 0
for rep in range(2):
    graph.replay()
    torch.cuda.synchronize()
    for name in ref:
        assert torch.equal(out[name], ref[name]), (rep, name)
print("first call under capture: ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    """The entry point's per-device set-up (the symbol lookup and the kernels' LDS attribute)
    on its first call in a fresh process, made while a HIP graph is being captured."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("\n[no-alloc] first call under capture (fresh process)", flush=True)
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, root], capture_output=True, text=True,
                       timeout=240, cwd=root)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "first call under capture: ok" in r.stdout
