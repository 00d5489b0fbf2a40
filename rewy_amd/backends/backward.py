"""Complete backward bindings on the gfx950 HIP kernels.

Same callables, keyword signatures and return tuples as the reference's
``backends/backward.py`` (``kda_backward`` :63-73, ``gdn2_backward`` :75-81,
``gdn_backward`` :133, ``delta_backward`` :136), which are keyword-compatible
with FLA's ``chunk_<op>_bwd``.  Each one runs

  1. (recompute policy) ``fdr_fwd_h_wy`` -- w (and qg, kg), h, v_new from the saved
     tensors, w / u formed inside the forward scan (``fdr_prepare_wu`` + ``fdr_fwd_h`` for a
     vector gate whose value tiles are narrower than 64, see ``ops.fwd_h_wy_pays``);
  2. ``fdr_state_bwd``  -- reverse state recurrence with dv_local = Aqk^T dO fused in (for
     the scalar / no-gate families Aqk formed in-kernel from q, k);
  3. ``fdr_chunk_bwd``  -- residual-WY products, dAqk, matrix intra, gate/beta
     epilogue and the in-chunk reverse cumsum of dg, one work-group per chunk.

When batch x heads is too small to fill the GPU and the sequence long, the two
recurrences run instead in affine-step form (after ``fdr_prepare_wu``: w, u and qg, kg or Aqk) (``ops.recurrences``,
``fdr_affine_*``): chunk-parallel step matrices, one scan launch carrying both
recurrences side by side, and a chunk-parallel pass for v_new and dR.
With 17 <= batch x heads <= 127, and on short rows at batch x heads <= 16, the recompute policy
runs the direct backward state recurrence and the direct forward scan side by side in one
launch (``fdr_paired_recurrences``), at a value-tile width that gives each at most half the
CUs (``ops.paired_tile``).
With a few more heads and long rows the recompute policy runs the forward scan
(``fdr_fwd_h``) on the current stream beside the segmented backward state recurrence
(``fdr_state_bwd_segmented``) on a second stream (``ops.side_by_side_pays``).

There is no fallback: a missing HIP library or an unsupported argument raises.
"""
from __future__ import annotations

import threading

import torch

from .. import ops

_UNSUPPORTED = ("cp_context",)


def _varlen(q, kw):
    """The packed variable-length batch of ``cu_seqlens`` (B = 1) as an ``ops.Varlen``, or None.

    Sequences start anywhere: every kernel takes the batch's chunk map (FLA's
    chunk_indices / chunk_offsets, derived here from cu_seqlens; a sequence's last chunk
    may be partial), and the state recurrences restart at every sequence's first chunk."""
    cu = kw.get("cu_seqlens")
    if cu is None:
        if kw.get("chunk_indices") is not None or kw.get("chunk_offsets") is not None:
            raise NotImplementedError("chunk_indices / chunk_offsets without cu_seqlens")
        return None
    B, T = q.shape[:2]
    if B != 1:
        raise ValueError(f"The batch size is expected to be 1 rather than {B} when using `cu_seqlens`.")
    vl = cu if isinstance(cu, ops.Varlen) else ops.Varlen(cu, q.device)
    if vl.T != T:
        raise ValueError("cu_seqlens must rise from 0 to T")
    return vl


def _check_common(kind, kw):
    for name in _UNSUPPORTED:
        if kw.get(name) is not None:
            raise NotImplementedError(f"{kind} HIP backward: {name} is not supported")
    if kw.get("chunk_size", 64) != 64:
        raise NotImplementedError(f"{kind} HIP backward: chunk_size must be 64")
    if kw.get("use_gate_in_kernel", False) and kind != "kda":
        raise NotImplementedError(f"{kind} HIP backward: use_gate_in_kernel is not supported")
    if kw.get("safe_gate", False):
        raise NotImplementedError(f"{kind} HIP backward: safe_gate is not supported")
    if kw.get("use_graph", False):
        raise NotImplementedError(f"{kind} HIP backward: use_graph is not supported")


def _bf(x):
    if x.dtype is torch.bfloat16 and x.is_contiguous():      # (the common case, without a call into torch)
        return x
    return x.to(torch.bfloat16).contiguous()


def _group_sum(out, HQ):
    """Grouped value heads: dq / dk come per value head; q / k's gradient is the sum over
    each head's group (FLA's head map i_h = i_hv // (HV / H)), formed in fp32 in one pass
    (fdr_group_sum)."""
    for n in ("dq", "dk"):
        x = out[n]
        if x.shape[2] != HQ:
            out[n] = ops.group_sum(x.contiguous(), HQ) if x.dtype == torch.bfloat16 else \
                x.view(*x.shape[:2], HQ, x.shape[2] // HQ, x.shape[3]).float().sum(3).to(x.dtype)
    return out


def _f32(x):
    if x is None or (x.dtype is torch.float32 and x.is_contiguous()):
        return x
    return x.to(torch.float32).contiguous()


_SIDE = {}
_SIDE_LOCK = threading.Lock()


def _side_by_side(first, second):
    """first() enqueued on the current stream while second() is enqueued on a side stream
    that waits only for the work enqueued before first(); the current stream then waits for
    the side stream.  For two independent recurrences that each leave most of the GPU idle
    (few heads, long rows: the forward scan of the recompute policy beside the segmented
    backward state recurrence).  first() is enqueued first so that its few long-lived
    work-groups are placed before second()'s launches fill the GPU (the other way round,
    the scan's work-groups waited for free CUs and the scan took 2.4x as long).  The tensors
    that second() returns are marked as used by the current stream.

    Lifetimes: second() reads tensors allocated on the current stream.  The join
    (``cur.wait_stream(side)``) is enqueued before this function returns, so memory that
    the caller frees afterwards can only be reused by work ordered after the side stream's
    kernels.  A caller must not free an input of second() before this function returns.
    The side streams are created once per device, under a lock."""
    cur = torch.cuda.current_stream()
    side = _SIDE.get(cur.device)
    if side is None:
        with _SIDE_LOCK:
            side = _SIDE.get(cur.device)
            if side is None:
                side = _SIDE[cur.device] = torch.cuda.Stream(cur.device)    # default priority
    side.wait_stream(cur)
    a = first()
    with torch.cuda.stream(side):
        b = second()
    cur.wait_stream(side)
    for t in b:
        if torch.is_tensor(t):
            t.record_stream(cur)
    return a, b


def _vector(op, q, k, v, gates, Aqk, Akk, scale, initial_state, do, dht, g, saved, gate_fold=None,
            beta_sigmoid=0.0, state_v_first=False, saved_h_v_first=None, **kw):
    """Shared vector-gate (KDA / GDN2) backward.  ``gate_fold``, ``beta_sigmoid``: see ops.chunk_bwd.
    ``state_v_first``: initial_state, dht and dh0 are [N,H,V,K], and so is a saved ``h``
    unless ``saved_h_v_first`` says otherwise (the kernels read and write those layouts)."""
    _check_common(op, kw)
    vf = bool(state_v_first)
    hvf = vf if saved_h_v_first is None else bool(saved_h_v_first)
    vl = _varlen(q, kw)
    q, k, v, do = _bf(q), _bf(k), _bf(v), _bf(do)
    g = _f32(g)
    Aqk, Akk = _f32(Aqk), _f32(Akk)
    recompute = saved.get("h") is None
    N, H, NT = (q.shape[0], v.shape[2], q.shape[1] // ops.CHUNK) if vl is None else (vl.N, v.shape[2], vl.NC)
    if recompute and vl is None and ops.paired_tile(N, H, NT, ops.GATE_VECTOR):
        # batch x heads too small for one direct recurrence to fill the GPU: the backward
        # state recurrence and the forward scan side by side, both direct, at a value-tile
        # width that gives each launch at most half the CUs
        vb = ops.paired_tile(N, H, NT, ops.GATE_VECTOR)
        fold_u = ops.PAIRED_U
        raw = fold_u and ops.PAIRED_RAW and vb == 64
        formw = raw and ops.PAIRED_FORMW and gates.get("b") is not None
        bgate = None if gates.get("b") is None else _bf(gates["b"])
        # (formw: w formed in both recurrences as well, so no prepare_wu at all)
        pre = (dict(w=None) if formw else
               _prepare_vector(k, v, g, Akk, gates, q, vl, want_u=not fold_u, want_qkg=not raw))

        def state():
            if raw:         # qg / kg (and w) formed as the state recurrence stages each chunk
                return ops.state_bwd(q, k, pre["w"], g, ops.GATE_VECTOR, do, scale, aqk=Aqk, dht=_f32(dht),
                                     want_dh0=initial_state is not None, value_block=vb, method="direct",
                                     state_v_first=vf, raw_qk=True, beta=_f32(gates.get("beta")), b=bgate,
                                     Akk=Akk)
            return _state_vector(pre, g, do, scale, Aqk, dht, initial_state, vl, vf, method="direct",
                                 value_block=vb)

        def scan():
            if fold_u:      # u (and kg, w) formed inside the scan
                return ops.fwd_h_u(k, pre["w"], v, Akk, g, ops.GATE_VECTOR, beta=_f32(gates.get("beta")),
                                   w_gate=None if gates.get("w") is None else _bf(gates["w"]), b=bgate,
                                   h0=_f32(initial_state), value_block=vb, state_v_first=vf,
                                   kg=None if raw else pre["kg"])
            return ops.fwd_h(pre["kg"], pre["w"], pre["u"], g, ops.GATE_VECTOR, h0=_f32(initial_state),
                             method="direct", value_block=vb, state_v_first=vf)
        if fold_u and ops.PAIRED_ONE_LAUNCH:
            # both in one launch (the same kernels' bodies, no second stream)
            (dh, dR, dh0), (h, v_new, _) = ops.paired_recurrences(
                q, k, pre["w"], g, ops.GATE_VECTOR, do, scale, v, Akk, vb, aqk=Aqk, beta=_f32(gates.get("beta")),
                b=bgate, w_gate=None if gates.get("w") is None else _bf(gates["w"]),
                qg=None if raw else pre["qg"], kg=None if raw else pre["kg"], raw_qk=raw, h0=_f32(initial_state),
                dht=_f32(dht), want_dh0=initial_state is not None, state_v_first=vf)
        else:
            (dh, dR, dh0), (h, v_new, _) = _side_by_side(state, scan)
        saved, hvf = dict(v_new=v_new, h=h), False
    elif recompute and vl is None and ops.affine_pays(v):
        # few heads: both recurrences side by side in affine-step form
        pre = _prepare_vector(k, v, g, Akk, gates, q, vl)
        h, v_new, dh, dR, dh0 = ops.recurrences(pre["qg"], pre["kg"], pre["w"], pre["u"], g, ops.GATE_VECTOR,
                                                do, scale, aqk=Aqk, h0=_f32(initial_state), dht=_f32(dht),
                                                want_dh0=initial_state is not None, state_v_first=vf)
        saved, hvf = dict(v_new=v_new, h=h), False
    elif recompute and (ops.side_by_side_pays(N, H, NT) if vl is None else
                        ops.SIDE_BY_SIDE and not ops.fwd_h_wy_pays(N, H, ops.GATE_VECTOR, vl)):
        # the forward scan on one stream beside the backward state recurrence on another:
        # few heads and long rows (the segmented recurrence), or a packed batch the fused
        # sweep does not take (its short sequences leave CUs idle while the longest runs)
        pre = _prepare_vector(k, v, g, Akk, gates, q, vl)
        (h, v_new, _), (dh, dR, dh0) = _side_by_side(
            lambda: ops.fwd_h(pre["kg"], pre["w"], pre["u"], g, ops.GATE_VECTOR, h0=_f32(initial_state),
                              method="direct", varlen=vl, state_v_first=vf),
            lambda: _state_vector(pre, g, do, scale, Aqk, dht, initial_state, vl, vf, method="segmented"))
        saved, hvf = dict(v_new=v_new, h=h), False
    else:
        if recompute:
            saved, hvf = _recompute_vector(q, k, v, g, Akk, initial_state, gates, vl, vf), False
        dh, dR, dh0 = _state_vector(saved, g, do, scale, Aqk, dht, initial_state, vl, vf)
    out = ops.chunk_bwd(q, k, v, _bf(saved["v_new"]), do, dR, g, ops.GATE_VECTOR, Akk,
                        _bf(saved["h"]), dh, scale, beta=_f32(gates.get("beta")),
                        b=None if gates.get("b") is None else _bf(gates["b"]),
                        w=None if gates.get("w") is None else _bf(gates["w"]),
                        gate_fold=gate_fold, beta_sigmoid=beta_sigmoid, h_v_first=hvf, varlen=vl)
    return _group_sum(out, q.shape[2]), dh0


def _state_vector(saved, g, do, scale, Aqk, dht, initial_state, vl=None, vf=False, method="auto", value_block=0):
    return ops.state_bwd(_bf(saved["qg"]), _bf(saved["kg"]), _bf(saved["w"]), g, ops.GATE_VECTOR, do, scale,
                         aqk=Aqk, dht=_f32(dht), want_dh0=initial_state is not None, value_block=value_block,
                         method=method if vl is None else "direct", varlen=vl, state_v_first=vf)


def _prepare_vector(k, v, g, Akk, gates, q, vl=None, want_u=True, want_qkg=True):
    b = None if gates.get("b") is None else _bf(gates["b"])
    w = None if gates.get("w") is None else _bf(gates["w"])
    return ops.prepare_wu(k, v, Akk, ops.GATE_VECTOR, g=g, beta=_f32(gates.get("beta")), b=b, w=w, q=q,
                          want_qkg=want_qkg, varlen=vl, want_u=want_u)


def _recompute_vector(q, k, v, g, Akk, initial_state, gates, vl=None, vf=False):
    """The recompute policy: w, qg, kg, h, v_new -- in one sweep (fdr_fwd_h_wy: w / u formed
    inside the forward scan, u never written) when that pays, else fdr_prepare_wu then fdr_fwd_h."""
    N = q.shape[0] if vl is None else vl.N
    if ops.fwd_h_wy_pays(N, v.shape[2], ops.GATE_VECTOR, vl):
        b = None if gates.get("b") is None else _bf(gates["b"])
        w = None if gates.get("w") is None else _bf(gates["w"])
        sw = ops.fwd_h_wy(k, v, Akk, g, ops.GATE_VECTOR, beta=_f32(gates.get("beta")), q=q, b=b, w=w,
                          h0=_f32(initial_state), varlen=vl, state_v_first=vf)
        return dict(w=sw["w"], qg=sw["qg"], kg=sw["kg"], v_new=sw["v_new"], h=sw["h"])
    pre = _prepare_vector(k, v, g, Akk, gates, q, vl)
    h, v_new, _ = ops.fwd_h(pre["kg"], pre["w"], pre["u"], g, ops.GATE_VECTOR, h0=_f32(initial_state),
                            method="direct", varlen=vl, state_v_first=vf)
    return dict(w=pre["w"], qg=pre["qg"], kg=pre["kg"], v_new=v_new, h=h)


def kda_backward(q, k, v, beta, Aqk, Akk, scale, initial_state, do, dht, g, g_org=None,
                 state_v_first=False, cu_seqlens=None, chunk_indices=None, chunk_size=64,
                 safe_gate=False, lower_bound=None, use_gate_in_kernel=False, A_log=None,
                 dt_bias=None, disable_recompute=False, cp_context=None, w=None, u=None, qg=None,
                 kg=None, v_new=None, h=None, use_graph=False, chunk_offsets=None, beta_sigmoid=0.0,
                 saved_h_v_first=None):
    """KDA backward -> (dq, dk, dv, db, dg, dh0, dA_log, ddt_bias).

    ``state_v_first``: initial_state, dht, dh0 and a saved h in FLA's [.., V, K] layout, read
    and written in place by the kernels.  ``saved_h_v_first`` (this build's addition, default:
    follow state_v_first) states the layout of the saved h separately.

    ``beta_sigmoid`` (this build's addition, default off): s > 0 when ``beta`` is
    s * sigmoid(beta_raw) activated in the forward; db is then dL/dbeta_raw, the fused
    beta-sigmoid backward of reference _compat/kda.py:204-205 done in the chunk kernel.

    ``cu_seqlens``: a packed batch (B = 1) whose sequences start anywhere, or the
    ``ops.Varlen`` chunk map built from it (the chunk Function passes the forward's)."""
    from ..runtime import record
    saved = dict(w=w, u=u, qg=qg, kg=kg, v_new=v_new, h=h)
    # the in-kernel gate's backward rides in the chunk kernel's dg stores (one pass fewer
    # over dg); g is the activated gate's cumsum, g_org the raw gate input (FLA convention)
    fold = (dict(g_raw=g_org, A_log=A_log, dt_bias=dt_bias, lower_bound=lower_bound)
            if use_gate_in_kernel else None)
    out, dh0 = _vector("kda", q, k, v, dict(beta=beta), Aqk, Akk, scale, initial_state, do, dht, g,
                       saved, gate_fold=fold, beta_sigmoid=beta_sigmoid, state_v_first=state_v_first,
                       saved_h_v_first=saved_h_v_first, cu_seqlens=cu_seqlens,
                       chunk_indices=chunk_indices, chunk_size=chunk_size, safe_gate=safe_gate,
                       use_gate_in_kernel=use_gate_in_kernel, cp_context=cp_context,
                       use_graph=use_graph, chunk_offsets=chunk_offsets)
    record("kda", "optimized_backward")
    dg, dA_log, ddt_bias = out["dg"], out.get("dA_log"), out.get("ddt_bias")
    return out["dq"], out["dk"], out["dv"], out["dbeta"], dg, dh0, dA_log, ddt_bias


def gdn2_backward(q, k, v, b, w_gate, Aqk, Akk, scale, initial_state, do, dht, g, g_org=None,
                  cu_seqlens=None, chunk_indices=None, chunk_size=64, safe_gate=False,
                  lower_bound=None, use_gate_in_kernel=False, A_log=None, dt_bias=None,
                  state_v_first=False, w_wy=None, u_wy=None, qg=None, kg=None, v_new=None, h=None,
                  disable_recompute=False, cp_context=None, saved_h_v_first=None):
    """GDN2 backward -> (dq, dk, dv, db, dw, dg, dh0, dA_log, ddt_bias).  ``state_v_first`` and
    ``saved_h_v_first`` as for kda_backward."""
    from ..runtime import record
    saved = dict(w=w_wy, u=u_wy, qg=qg, kg=kg, v_new=v_new, h=h)
    out, dh0 = _vector("gdn2", q, k, v, dict(b=b, w=w_gate), Aqk, Akk, scale, initial_state, do, dht,
                       g, saved, state_v_first=state_v_first, saved_h_v_first=saved_h_v_first, cu_seqlens=cu_seqlens,
                       chunk_indices=chunk_indices, chunk_size=chunk_size, safe_gate=safe_gate,
                       use_gate_in_kernel=use_gate_in_kernel, cp_context=cp_context)
    record("gdn2", "optimized_backward")
    return out["dq"], out["dk"], out["dv"], out["db"], out["dw"], out["dg"], dh0, None, None


def _scalar(op, q, k, v, beta, A, scale, initial_state, do, dht, g, beta_sigmoid=0.0, state_v_first=False, **kw):
    """GDN / DeltaNet: recompute w, u, h, v_new, then the state and chunk kernels
    (reference ``_scalar``, backends/backward.py:96-131)."""
    from ..runtime import record
    _check_common(op, kw)
    vl = _varlen(q, kw)
    q, k, v, do = _bf(q), _bf(k), _bf(v), _bf(do)
    g = _f32(g)
    A = _f32(A)
    beta = _f32(beta)
    gate = ops.GATE_SCALAR if op == "gdn" else ops.GATE_NONE
    affine = vl is None and q.shape[2] == v.shape[2] and ops.affine_pays(v)
    # mid-size batch x heads: the direct recurrences side by side (ops.paired_tile)
    vb = 0 if vl is not None else ops.paired_tile(q.shape[0], v.shape[2], q.shape[1] // ops.CHUNK, gate)
    # the direct state recurrence forms Aqk itself from the raw q / k it stages; w and u are then
    # formed inside the forward scan's sweep where that pays (fdr_fwd_h_wy: u never leaves the
    # chip), else by fdr_prepare_wu without Aqk
    inline = vb > 0 or (not affine and (vl is not None or ops.state_form(q.shape[0], v.shape[2],
                                                                          q.shape[1] // ops.CHUNK) == "direct"))
    if vb and ops.PAIRED_U and ops.PAIRED_ONE_LAUNCH and ops.SCALAR_ONE_CALL:
        # the paired form below as one library call (fdr_scalar_bwd: the same launches, the same
        # bits, a third of the host time)
        out, dh0 = ops.scalar_bwd(q, k, v, g, gate, beta, A, do, scale, vb, vb <= ops.PAIRED_AQK_MAX_VB,
                                  dht=_f32(dht), h0=_f32(initial_state), want_dh0=initial_state is not None,
                                  beta_sigmoid=beta_sigmoid, state_v_first=state_v_first)
        record(op, "optimized_backward")
        return _group_sum(out, q.shape[2]), dh0
    if inline:
        pre = None
        if not vb and ops.fwd_h_wy_pays(q.shape[0] if vl is None else vl.N, v.shape[2], gate, vl):
            sw = ops.fwd_h_wy(k, v, A, g, gate, beta=beta, h0=_f32(initial_state), varlen=vl,
                              state_v_first=state_v_first)
            w, h, v_new = sw["w"], sw["h"], sw["v_new"]
        else:
            # paired (vb): u formed inside the scan where ops.PAIRED_U holds; at narrow value tiles
            # Aqk written here for the state recurrence (ops.PAIRED_AQK_MAX_VB)
            aqk_pre = 0 < vb <= ops.PAIRED_AQK_MAX_VB
            pre = ops.prepare_wu(k, v, A, gate, g=g, beta=beta, varlen=vl, want_u=not (vb and ops.PAIRED_U),
                                 q=q if aqk_pre else None, want_aqk=aqk_pre, scale=scale)
            w = pre["w"]

        def state():
            return ops.state_bwd(q, k, w, g, gate, do, scale, aqk=None if pre is None else pre.get("Aqk"),
                                 dht=_f32(dht), want_dh0=initial_state is not None, method="direct", varlen=vl,
                                 state_v_first=state_v_first, value_block=vb)

        def scan():
            if pre["u"] is None:
                return ops.fwd_h_u(k, w, v, A, g, gate, beta=beta, h0=_f32(initial_state), value_block=vb,
                                   state_v_first=state_v_first)
            return ops.fwd_h(k, w, pre["u"], g, gate, h0=_f32(initial_state), method="direct", varlen=vl,
                             state_v_first=state_v_first, value_block=vb)
        if pre is None:
            dh, dR, dh0 = state()
        elif vb and pre["u"] is None and ops.PAIRED_ONE_LAUNCH:
            # both recurrences in one launch (the same kernels' bodies, no second stream)
            (dh, dR, dh0), (h, v_new, _) = ops.paired_recurrences(
                q, k, w, g, gate, do, scale, v, A, vb, aqk=pre.get("Aqk"), beta=beta, h0=_f32(initial_state),
                dht=_f32(dht), want_dh0=initial_state is not None, state_v_first=state_v_first)
        elif vb:
            # the state recurrence (the longer chain) first, the scan on the side stream
            (dh, dR, dh0), (h, v_new, _) = _side_by_side(state, scan)
        elif vl is not None and ops.SIDE_BY_SIDE:
            # a packed batch: its short sequences leave CUs idle while the longest runs
            (h, v_new, _), (dh, dR, dh0) = _side_by_side(scan, state)
        else:
            h, v_new, _ = scan()
            dh, dR, dh0 = state()
        out = _group_sum(ops.chunk_bwd(q, k, v, v_new, do, dR, g, gate, A, h, dh, scale, beta=beta,
                                       beta_sigmoid=beta_sigmoid, varlen=vl), q.shape[2])
        record(op, "optimized_backward")
        return out, dh0
    pre = ops.prepare_wu(k, v, A, gate, g=g, beta=beta, q=q, want_aqk=True, scale=scale, varlen=vl)
    if affine:
        # few heads: both recurrences side by side in affine-step form
        h, v_new, dh, dR, dh0 = ops.recurrences(q, k, pre["w"], pre["u"], g, gate, do, scale, aqk=pre["Aqk"],
                                                h0=_f32(initial_state), dht=_f32(dht),
                                                want_dh0=initial_state is not None, state_v_first=state_v_first)
    else:
        # (grouped q / k heads take the direct state recurrence)
        sbs = (vl is None and q.shape[2] == v.shape[2]
               and ops.side_by_side_pays(q.shape[0], v.shape[2], q.shape[1] // ops.CHUNK))
        method = "segmented" if sbs else "auto"

        def scan():
            return ops.fwd_h(k, pre["w"], pre["u"], g, gate, h0=_f32(initial_state), method="direct",
                             varlen=vl, state_v_first=state_v_first)

        def state():
            return ops.state_bwd(q, k, pre["w"], g, gate, do, scale, aqk=pre["Aqk"], dht=_f32(dht),
                                 want_dh0=initial_state is not None, method=method, varlen=vl,
                                 state_v_first=state_v_first)
        if sbs:
            (h, v_new, _), (dh, dR, dh0) = _side_by_side(scan, state)
        else:
            h, v_new, _ = scan()
            dh, dR, dh0 = state()
    out = _group_sum(ops.chunk_bwd(q, k, v, v_new, do, dR, g, gate, A, h, dh, scale, beta=beta,
                                   beta_sigmoid=beta_sigmoid, varlen=vl), q.shape[2])
    record(op, "optimized_backward")
    return out, dh0


def _aqk_scalar(q, k, g, scale):
    """Intra-chunk scores scale * tril(q k^T 2^(g_i - g_j)) for scalar/no gates."""
    from ..forward import from_chunks, to_chunks
    qc, kc = to_chunks(q.float()), to_chunks(k.float())
    s = scale * qc @ kc.transpose(-1, -2)
    C = s.shape[-1]
    low = torch.tril(torch.ones(C, C, dtype=torch.bool, device=q.device))
    if g is not None:
        gc = to_chunks(g)
        d = gc[..., :, None] - gc[..., None, :]
        s = s * torch.exp2(torch.where(low, d, torch.full_like(d, -float("inf"))))
    s = torch.where(low, s, torch.zeros((), device=q.device))
    return from_chunks(s)


def gdn_backward(q, k, v, g, beta, A, scale, initial_state, do, dht, **kw):
    """GDN backward -> (dq, dk, dv, db, dg, dh0, None, None)."""
    out, dh0 = _scalar("gdn", q, k, v, beta, A, scale, initial_state, do, dht, g, **kw)
    return out["dq"], out["dk"], out["dv"], out["dbeta"], out["dg"], dh0, None, None


def delta_backward(q, k, v, beta, A, scale, initial_state, do, dht, **kw):
    """DeltaNet backward -> (dq, dk, dv, db, dh0)."""
    out, dh0 = _scalar("delta", q, k, v, beta, A, scale, initial_state, do, dht, None, **kw)
    return out["dq"], out["dk"], out["dv"], out["dbeta"], dh0
