"""Autograd contract and public ``chunk_*`` operators for both backends.

One autograd Function serves the four families.  Its forward is the HIP
forward (``rewy_amd.hip_forward``) for the optimized backend on a GPU and the
PyTorch restatement (``rewy_amd.forward``) otherwise; it saves FLA's tensor list
(reference ``_compat/kda.py:120-144``: q, k, v, g_cumsum, beta, Aqk, Akk and,
under full saving, w, u, qg, kg, v_new, h).  Its backward is chosen when the
forward runs and stays bound to the Function afterwards (reference
``docs/architecture.md``: "Its own autograd Function permanently selects its
backward"):

* ``optimized`` -> ``rewy_amd.backends.backward`` (HIP kernels, no fallback);
* ``original``  -> ``rewy_amd.original.original_backward`` (PyTorch ops).

The public functions keep the reference's signatures (``_compat/kda.py:214``,
``_compat/gdn.py`` ``chunk_gated_delta_rule``, ``_compat/gdn2.py:205``,
``_compat/delta.py``) and argument checks; options outside this build's
envelope raise ``NotImplementedError``.
"""
from __future__ import annotations

import torch

from ..forward import chunk_forward


def _l2norm(x, backend):
    """q / k normalisation: HIP kernels for the optimized backend on a GPU, torch ops otherwise."""
    from ..norm import l2norm
    return l2norm(x, native=backend == "optimized" and x.is_cuda)


class ChunkFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, op, backend, full_saving, scale, output_final_state, q, k, v, g, beta, b, w,
                initial_state, cu_seqlens=None, gate=None, A_log=None, dt_bias=None, beta_act=None,
                state_v_first=False):
        # cu_seqlens (optimized backend on a GPU only): B = 1 holds sequences packed along T,
        # starting anywhere; every kernel takes the batch's chunk map and the state scans
        # restart at each sequence.
        # gate = (lower_bound,) (KDA, optimized backend on a GPU, no padded tokens): g is the
        # raw gate, activated here by the HIP gate kernel; its backward, with dA_log and
        # ddt_bias, is folded into the chunk kernel.
        # beta_act = s (scalar-beta families, optimized backend on a GPU): beta is the raw
        # input, activated here as s * sigmoid(beta); its backward rides in the chunk
        # kernel's dbeta stores.
        # state_v_first (optimized backend on a GPU): initial / final states are [N,H,V,K],
        # read and written so by the kernels.
        native = backend == "optimized" and q.is_cuda
        if state_v_first and not native:
            raise ValueError("V-first states in the chunk Function are the optimized GPU path's")
        if gate is not None and not (native and op == "kda"):
            raise ValueError("the folded gate is the optimized GPU path's (KDA)")
        if beta_act is not None and not (native and op != "gdn2"):
            raise ValueError("the folded beta sigmoid is the optimized GPU path's (scalar beta)")
        ctx.gate, ctx.beta_act, ctx.vf = gate, beta_act, bool(state_v_first)
        ctx.g_dtype = None if g is None else g.dtype
        ctx.beta_dtype = None if beta is None else beta.dtype
        g_raw = None
        if gate is not None:
            from ..gates import kda_gate
            g_raw, g = g, kda_gate(g, A_log, dt_bias, gate[0], native=True)
        if beta_act is not None:
            from ..gates import beta_sigmoid
            beta = beta_sigmoid(beta, beta_act, native=True)
        if backend == "optimized" and q.is_cuda:
            from ..hip_forward import chunk_forward_hip
            from ..ops import Varlen
            varlen = None if cu_seqlens is None else Varlen(cu_seqlens, q.device)
            ctx.cu_seqlens = varlen            # the chunk map, reused by the backward
            o, final, sv = chunk_forward_hip(op, q, k, v, g=g, beta=beta, b=b, w=w,
                                             initial_state=initial_state, scale=scale,
                                             output_final_state=output_final_state, varlen=varlen,
                                             state_v_first=state_v_first)
        elif cu_seqlens is not None:
            raise NotImplementedError("packed cu_seqlens batches in the chunk Function are the optimized GPU path's")
        else:
            ctx.cu_seqlens = None
            o, final, sv = chunk_forward(op, q, k, v, g=g, beta=beta, b=b, w=w,
                                         initial_state=initial_state, scale=scale,
                                         output_final_state=output_final_state)
        keep = full_saving and op in ("kda", "gdn2")
        ctx.save_for_backward(q, k, v, sv["gc"], beta, b, w, sv["Aqk"], sv["Akk"], initial_state,
                              *(sv[n] if keep else None for n in ("w", "u", "qg", "kg", "v_new", "h")),
                              g_raw, A_log, dt_bias)
        ctx.op, ctx.backend, ctx.scale = op, backend, scale
        ctx.has_h0 = initial_state is not None
        return o, final

    @staticmethod
    def backward(ctx, do, dht):
        (q, k, v, gc, beta, b, w, Aqk, Akk, h0, w_wy, u_wy, qg, kg, v_new, h, g_raw, A_log,
         dt_bias) = ctx.saved_tensors
        dA_log = ddt_bias = None
        op, scale = ctx.op, ctx.scale
        if ctx.backend == "optimized":
            from ..backends import backward as bw
            cu = ctx.cu_seqlens
            bsig = ctx.beta_act or 0.0
            # the saved per-chunk h is this package's [B,NT,H,K,V] whatever the state layout
            lay = dict(state_v_first=ctx.vf, saved_h_v_first=False) if ctx.vf else {}
            if op == "kda":
                gate_kw = {} if ctx.gate is None else dict(
                    use_gate_in_kernel=True, g_org=g_raw, A_log=A_log, lower_bound=ctx.gate[0],
                    dt_bias=None if dt_bias is None else dt_bias.reshape(-1))
                dq, dk, dv, db, dg, dh0, dA_log, ddt_bias = bw.kda_backward(
                    q=q, k=k, v=v, beta=beta, Aqk=Aqk, Akk=Akk, scale=scale, initial_state=h0,
                    do=do, dht=dht, g=gc, w=w_wy, u=u_wy, qg=qg, kg=kg, v_new=v_new, h=h, cu_seqlens=cu,
                    beta_sigmoid=bsig, **lay, **gate_kw)
                dw = None
            elif op == "gdn2":
                dq, dk, dv, db, dw, dg, dh0, _, _ = bw.gdn2_backward(
                    q=q, k=k, v=v, b=b, w_gate=w, Aqk=Aqk, Akk=Akk, scale=scale, initial_state=h0,
                    do=do, dht=dht, g=gc, w_wy=w_wy, u_wy=u_wy, qg=qg, kg=kg, v_new=v_new, h=h,
                    cu_seqlens=cu, **lay)
            elif op == "gdn":
                dq, dk, dv, db, dg, dh0, _, _ = bw.gdn_backward(
                    q=q, k=k, v=v, g=gc, beta=beta, A=Akk, scale=scale, initial_state=h0, do=do, dht=dht,
                    cu_seqlens=cu, beta_sigmoid=bsig, state_v_first=ctx.vf)
                dw = None
            else:
                dq, dk, dv, db, dh0 = bw.delta_backward(
                    q=q, k=k, v=v, beta=beta, A=Akk, scale=scale, initial_state=h0, do=do, dht=dht,
                    cu_seqlens=cu, beta_sigmoid=bsig, state_v_first=ctx.vf)
                dg = dw = None
        else:
            from ..original import original_backward
            saved = None if h is None else dict(w=w_wy, u=u_wy, qg=qg, kg=kg, v_new=v_new, h=h)
            out = original_backward(op, q, k, v, gc, Akk, scale, h0, do, dht, beta=beta, b=b, w=w,
                                    Aqk=Aqk if op in ("kda", "gdn2") else None, saved=saved)
            dq, dk, dv, dg, dh0 = out["dq"], out["dk"], out["dv"], out["dg"], out["dh0"]
            db = out["db"] if op == "gdn2" else out["dbeta"]
            dw = out["dw"]
        if not ctx.has_h0:
            dh0 = None
        cast = lambda x, ref: None if x is None or ref is None else x.to(ref.dtype)
        gb = cast(db, b) if op == "gdn2" else (None if db is None else db.to(ctx.beta_dtype))
        return (None, None, None, None, None, cast(dq, q), cast(dk, k), cast(dv, v),
                None if dg is None else dg.to(ctx.g_dtype),
                None if op == "gdn2" else gb, gb if op == "gdn2" else None, cast(dw, w), dh0, None, None,
                cast(dA_log, A_log), None if ddt_bias is None else ddt_bias.reshape(dt_bias.shape).to(dt_bias.dtype),
                None, None)


def _unsupported(name, **flags):
    for key, value in flags.items():
        if value:
            raise NotImplementedError(f"{name}: {key} is not supported by this build")


def _pad_time(xs, T):
    """Zero-pad the time axis of [B,T,...] tensors up to a multiple of 64.  Zero
    keys/values/gates leave the state untouched, so outputs of real tokens are
    unchanged (used by the original backend for arbitrary T)."""
    Tp = (T + 63) // 64 * 64
    if Tp == T:
        return xs, T
    out = []
    for x in xs:
        if x is None:
            out.append(None)
            continue
        pad = [0, 0] * (x.ndim - 2) + [0, Tp - T]
        out.append(torch.nn.functional.pad(x, pad))
    return out, Tp


def _run(op, backend, full_saving, scale, output_final_state, q, k, v, g, beta, b, w, h0, vf=False):
    T = q.shape[1]
    extra = (None, None, None, None, None, vf)
    if T % 64:
        (q, k, v, g, beta, b, w), _ = _pad_time((q, k, v, g, beta, b, w), T)
        o, final = ChunkFunction.apply(op, backend, full_saving, scale, output_final_state,
                                       q, k, v, g, beta, b, w, h0, *extra)
        return o[:, :T], final
    return ChunkFunction.apply(op, backend, full_saving, scale, output_final_state, q, k, v, g,
                               beta, b, w, h0, *extra)


def _unpack(x, bounds, Tp):
    """Packed [1, T, ...] -> [N, Tp, ...], each sequence zero-padded to Tp."""
    if x is None:
        return None
    rows = []
    for s, e in bounds:
        seq = x[:, s:e]
        pad = [0, 0] * (x.ndim - 2) + [0, Tp - (e - s)]
        rows.append(torch.nn.functional.pad(seq, pad))
    return torch.cat(rows, 0)


def _apply(op, backend, full_saving, scale, output_final_state, q, k, v, g, beta, b, w, h0,
           state_v_first=False, cu_seqlens=None, cu_seqlens_cpu=None, gate_fold=None, beta_act=None):
    """Layout adapters around the chunk Function (all autograd-transparent torch ops):

    * grouped value heads (HV = v.shape[2] > H): the optimized GPU path hands q and k
      over with their H heads and the kernels map value head i_hv to q / k head
      i_hv // (HV / H) (FLA's head map; dq / dk summed over each group); the torch paths
      repeat q and k over each group;
    * ``state_v_first``: initial / final states are [N, HV, V, K] at the boundary;
    * ``cu_seqlens`` (B = 1, packed): on the optimized backend on a GPU the kernels take
      the packed batch as it is, whatever the sequence lengths (each sequence's last chunk
      may be partial; its missing rows read as zero and are never written; the state
      scans restart at each sequence: work scales with the sum of the lengths);
      otherwise each sequence is zero-padded to the longest one and run as one batch
      row.  Zero keys, values and log-gates leave the state untouched, so outputs,
      final states and gradients of the real tokens are exact; padded positions are
      dropped.

    ``gate_fold`` = (lower_bound, A_log, dt_bias) (KDA's raw gate) and ``beta_act`` = s
    (raw beta, activated as s * sigmoid): on the optimized backend on a GPU the
    activations run inside the chunk Function and their backward rides in the chunk
    kernel; otherwise they run here as autograd nodes of their own (padded tokens must keep
    zero activated gates)."""
    H, HV = q.shape[2], v.shape[2]
    native = backend == "optimized" and q.is_cuda
    bounds = None
    if cu_seqlens is not None:
        if q.shape[0] != 1:
            raise ValueError(f"The batch size is expected to be 1 rather than {q.shape[0]} when using `cu_seqlens`.")
        # The chunk map is built on the host, as FLA's prepare_chunk_indices(cu_seqlens, chunk,
        # cu_seqlens_cpu) builds it (reference _compat/gdn.py:166): a caller that passes
        # cu_seqlens_cpu spares the one device-to-host copy of cu_seqlens per call, which the
        # map's construction otherwise needs.
        cu = (cu_seqlens_cpu if cu_seqlens_cpu is not None else cu_seqlens).tolist()
        bounds = list(zip(cu[:-1], cu[1:]))
        if h0 is not None and h0.shape[0] != len(bounds):
            raise ValueError(f"The number of initial states is expected to be equal to the number of input "
                             f"sequences, i.e., {len(bounds)} rather than {h0.shape[0]}.")
    # no padded tokens anywhere: dense rows of whole chunks, or a packed batch (native)
    unpadded = native and (cu_seqlens is not None or q.shape[1] % 64 == 0)
    if gate_fold is not None and not unpadded:
        from ..gates import KDAGate
        lb, A_log, dt_bias = gate_fold
        g = KDAGate.apply(g, A_log, dt_bias, lb, native)
        gate_fold = None
    if beta_act is not None and not unpadded:
        from ..gates import beta_sigmoid
        beta = beta_sigmoid(beta, beta_act, native=False)
        beta_act = None
    if HV != H:
        if HV % H:
            raise ValueError(f"num_v_heads (HV={HV}) must be divisible by num_qk_heads (H={H})")
        if not (native and op in ("kda", "gdn", "delta")):
            # the torch paths (and GDN2) take one q / k head per value head
            q = q.repeat_interleave(HV // H, dim=2)
            k = k.repeat_interleave(HV // H, dim=2)
            if b is not None:
                b = b.repeat_interleave(HV // H, dim=2)
    # V-first states: read and written in that layout by the kernels on the optimized GPU
    # path; transposed here for the torch paths
    vf = bool(state_v_first) and native
    if state_v_first and not vf and h0 is not None:
        h0 = h0.transpose(-1, -2)
    fold = (None, None, None) if gate_fold is None else ((gate_fold[0],), gate_fold[1], gate_fold[2])
    if cu_seqlens is None:
        if unpadded:
            o, final = ChunkFunction.apply(op, backend, full_saving, scale, output_final_state, q, k, v, g, beta, b,
                                           w, h0, None, *fold, beta_act, vf)
        else:
            o, final = _run(op, backend, full_saving, scale, output_final_state, q, k, v, g, beta, b, w, h0, vf)
    elif unpadded:
        # packed natively: the kernels take the batch as it is
        o, final = ChunkFunction.apply(op, backend, full_saving, scale, output_final_state, q, k, v, g, beta,
                                       b, w, h0, torch.tensor(cu, dtype=torch.int64), *fold, beta_act, vf)
    else:
        Tp = max(64, -(-max(e - s for s, e in bounds) // 64) * 64)
        xs = [_unpack(x, bounds, Tp) for x in (q, k, v, g, beta, b, w)]
        o, final = _run(op, backend, full_saving, scale, output_final_state, *xs, h0)
        o = torch.cat([o[i:i + 1, :e - s] for i, (s, e) in enumerate(bounds)], 1)
    if state_v_first and not vf and final is not None:
        final = final.transpose(-1, -2)
    return o, final


def make_kda(backend):
    def chunk_kda(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
                  use_qk_l2norm_in_kernel=False, use_gate_in_kernel=False,
                  use_beta_sigmoid_in_kernel=False, allow_neg_eigval=False, safe_gate=False,
                  lower_bound=None, disable_recompute=False, return_intermediate_states=False,
                  state_v_first=False, cu_seqlens=None, cu_seqlens_cpu=None, cp_context=None,
                  use_graph=False, max_num_seqs=None, **kwargs):
        """Kimi Delta Attention (per-channel vector gate); reference _compat/kda.py:214."""
        _unsupported("chunk_kda", return_intermediate_states=return_intermediate_states,
                     cp_context=cp_context is not None, use_graph=use_graph)
        if kwargs.get("chunk_size", 64) != 64:
            raise ValueError("`chunk_size` must be 64 for this build")
        A_log = dt_bias = None
        if use_gate_in_kernel:
            A_log, dt_bias = kwargs.get("A_log"), kwargs.get("dt_bias")
            if A_log is None and lower_bound is None:
                raise ValueError("`A_log` must be provided when `use_gate_in_kernel=True` and `lower_bound` is not set.")
        if safe_gate and use_gate_in_kernel:
            if lower_bound is None:
                raise ValueError("`lower_bound` must be specified when `safe_gate=True` and `use_gate_in_kernel=True`.")
            if not (-5 <= lower_bound < 0):
                raise ValueError(f"`lower_bound` must be in the safe range [-5, 0), got {lower_bound}.")
        if allow_neg_eigval and not use_beta_sigmoid_in_kernel:
            raise ValueError("`allow_neg_eigval=True` requires `use_beta_sigmoid_in_kernel=True`.")
        if initial_state is not None:
            assert initial_state.dtype == torch.float32, "initial_state must be in float32."
        B, T, H, K = q.shape
        HV = v.shape[2]
        assert q.shape == k.shape, f"q and k must have the same shape, got q={q.shape} vs k={k.shape}"
        assert HV % H == 0, f"For GVA, num_v_heads (HV={HV}) must be evenly divisible by num_qk_heads (H={H})"
        assert g.shape == (B, T, HV, K), f"g must have shape [B, T, HV, K]={[B, T, HV, K]}, got {list(g.shape)}"
        assert beta.shape == (B, T, HV), f"beta must have shape [B, T, HV]={[B, T, HV]}, got {list(beta.shape)}"
        if use_qk_l2norm_in_kernel:
            q, k = _l2norm(q, backend), _l2norm(k, backend)
        beta_act = (2.0 if allow_neg_eigval else 1.0) if use_beta_sigmoid_in_kernel else None
        if beta_act is not None and backend != "optimized":
            beta, beta_act = beta.sigmoid() * beta_act, None
        fold = None
        if use_gate_in_kernel:
            if backend == "optimized":
                # the activation runs inside the chunk Function where no token is padded,
                # its backward (dg_raw, dA_log, ddt_bias) riding in the chunk kernel
                fold = (lower_bound, A_log, dt_bias)
            else:
                # the fused activation as its own autograd node: g's gradient flows to
                # g_raw, A_log and dt_bias (torch expressions)
                from ..gates import KDAGate
                g = KDAGate.apply(g, A_log, dt_bias, lower_bound, False)
        scale = K ** -0.5 if scale is None else scale
        return _apply("kda", backend, disable_recompute, scale, output_final_state, q, k, v, g, beta,
                      None, None, initial_state, state_v_first=state_v_first, cu_seqlens=cu_seqlens,
                      cu_seqlens_cpu=cu_seqlens_cpu, gate_fold=fold, beta_act=beta_act)
    return chunk_kda


def make_gdn(backend):
    def chunk_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None,
                               output_final_state=False, use_qk_l2norm_in_kernel=False,
                               use_beta_sigmoid_in_kernel=False, allow_neg_eigval=False,
                               state_v_first=False, cu_seqlens=None, cu_seqlens_cpu=None,
                               chunk_indices=None, cp_context=None, **kwargs):
        """Gated DeltaNet (scalar gate); reference _compat/gdn.py chunk_gated_delta_rule."""
        _unsupported("chunk_gated_delta_rule", cp_context=cp_context is not None,
                     use_gate_in_kernel=kwargs.get("use_gate_in_kernel", False))
        if kwargs.get("chunk_size", 64) != 64:
            raise ValueError("`chunk_size` must be 64 for this build")
        if initial_state is not None:
            assert initial_state.dtype == torch.float32, "initial_state must be in float32."
        B, T, H, K = q.shape
        HV = v.shape[2]
        assert HV % H == 0, f"num_v_heads (HV={HV}) must be divisible by num_qk_heads (H={H})"
        assert g.shape == (B, T, HV), f"g must have shape [B, T, HV], got {list(g.shape)}"
        if use_qk_l2norm_in_kernel:
            q, k = _l2norm(q, backend), _l2norm(k, backend)
        beta_act = (2.0 if allow_neg_eigval else 1.0) if use_beta_sigmoid_in_kernel else None
        if beta_act is not None and backend != "optimized":
            beta, beta_act = beta.sigmoid() * beta_act, None
        scale = K ** -0.5 if scale is None else scale
        return _apply("gdn", backend, False, scale, output_final_state, q, k, v, g, beta, None, None,
                      initial_state, state_v_first=state_v_first, cu_seqlens=cu_seqlens,
                      cu_seqlens_cpu=cu_seqlens_cpu, beta_act=beta_act)
    return chunk_gated_delta_rule


def make_gdn2(backend):
    def chunk_gdn2(q, k, v, g, b, w, scale=None, initial_state=None, output_final_state=False,
                   use_qk_l2norm_in_kernel=False, use_gate_in_kernel=False, cu_seqlens=None,
                   cu_seqlens_cpu=None, safe_gate=False, lower_bound=None, disable_recompute=False,
                   return_intermediate_states=False, state_v_first=False, cp_context=None, **kwargs):
        """Gated DeltaNet 2 (vector gate, channel-wise erase b and write w gates);
        reference _compat/gdn2.py:205."""
        _unsupported("chunk_gdn2", use_gate_in_kernel=use_gate_in_kernel, safe_gate=safe_gate,
                     return_intermediate_states=return_intermediate_states,
                     cp_context=cp_context is not None)
        if kwargs.get("chunk_size", 64) != 64:
            raise ValueError("`chunk_size` must be 64 for GDN-2")
        if initial_state is not None:
            assert initial_state.dtype == torch.float32, "initial_state must be in float32."
        assert q.shape == k.shape == g.shape, "q, k, g must have the same shape."
        assert b.shape == q.shape, "b (channel-wise erase gate) must have shape [B, T, H, K]"
        assert w.shape == v.shape, "w (channel-wise write gate) must have shape [B, T, H, V]"
        if use_qk_l2norm_in_kernel:
            q, k = _l2norm(q, backend), _l2norm(k, backend)
        scale = k.shape[-1] ** -0.5 if scale is None else scale
        return _apply("gdn2", backend, disable_recompute, scale, output_final_state, q, k, v, g, None,
                      b, w, initial_state, state_v_first=state_v_first, cu_seqlens=cu_seqlens,
                      cu_seqlens_cpu=cu_seqlens_cpu)
    return chunk_gdn2


def make_delta(backend):
    def chunk_delta_rule(q, k, v, beta, scale=None, initial_state=None, output_final_state=False,
                         use_qk_l2norm_in_kernel=False, cu_seqlens=None, cu_seqlens_cpu=None,
                         **kwargs):
        """DeltaNet (no gate); reference _compat/delta.py chunk_delta_rule."""
        if "head_first" in kwargs:
            raise DeprecationWarning("head_first has been removed. Inputs must be in `[B, T, H, ...]` format.")
        if kwargs.get("chunk_size", 64) != 64:
            raise ValueError("`chunk_size` must be 64 for this build")
        assert q.dtype == k.dtype == v.dtype
        assert len(beta.shape) == 3, "beta must be of shape (batch size, seq len, num of head)."
        if use_qk_l2norm_in_kernel:
            q, k = _l2norm(q, backend), _l2norm(k, backend)
        scale = k.shape[-1] ** -0.5 if scale is None else scale
        return _apply("delta", backend, False, scale, output_final_state, q, k, v, None, beta, None,
                      None, initial_state, cu_seqlens=cu_seqlens, cu_seqlens_cpu=cu_seqlens_cpu)
    return chunk_delta_rule
