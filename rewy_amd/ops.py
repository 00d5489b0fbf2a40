"""Host wrappers of the HIP entry points: validate, allocate outputs, launch on
the current stream.

Each wrapper checks dtype, device, contiguity and shape of every operand on
the host before anything is enqueued, so a launch never sees an operand the
kernel's indexing does not assume.
"""
from __future__ import annotations

import torch

from . import _lib

GATE_NONE, GATE_SCALAR, GATE_VECTOR = 0, 1, 2
K_SUPPORTED = V_SUPPORTED = 128
CHUNK = 64


def _need(x, name, dtype, shape, device):
    # the common case in one test (tiny backwards validate ~20 operands per call)
    if x is not None and x.dtype is dtype and x.shape == shape and x.device == device and x.is_contiguous():
        return x
    if x is None:
        raise ValueError(f"{name} is required")
    if x.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {x.dtype}")
    if tuple(x.shape) != tuple(shape):
        raise ValueError(f"{name}: expected shape {tuple(shape)}, got {tuple(x.shape)}")
    if x.device != device:
        raise ValueError(f"{name}: expected device {device}, got {x.device}")
    if not x.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return x


# Affine-step recurrences pay off when B*H work-groups leave the GPU idle: the
# direct kernels are then bound by their per-chunk latency.
AFFINE_MAX_BH = 16
AFFINE_MIN_CHUNKS = 8
# ... for the backward state recurrence alone (full saving: no forward scan beside it), from
# more chunks: up to 16 the direct kernel's two launches fewer outweigh its longer steps
# (graph replay, KDA: B=1 H=4 8 chunks 33.2 vs 37.6 us, 12 chunks 39.4 vs 41.5, 16 chunks 45.6 vs
# 45.7; H=16 8 chunks 37.0 vs 42.6, 16 chunks 51.5 vs 53.7; GDN2 alike; 32 chunks the affine-step
# form, 57.2 vs 74.3 and 89.4 vs 91.8)
AFFINE_STATE_MIN_CHUNKS = 17
AFFINE_VALUE_BLOCK = 16


# Segmented state recurrence (fdr_state_bwd_segmented): long rows whose B*H value-tile
# work-groups leave most of the GPU idle.  Segments are sized so that the per-segment
# maps fill the chip (P and Q tiles: 4 work-groups per segment-head at 64-wide tiles).
SEG_MIN_CHUNKS = 256
# ... up to this B*H (exclusive): from B*H = 48 the direct recurrence at its 64-wide default tiles
# is faster however long the rows (KDA gate, graph replay, us, direct / segmented: B=1 T=16384
# H=32 550 / 540, H=48 641 / 896, H=64 649 / 950, H=96 895 / 1746; T=32768 H=40 1254 / 1252,
# H=80 1743 / 3434)
SEG_MAX_BH = 48
SEG_TARGET_GROUPS = 512
SEG_MIN_LEN = 16
# ... and from fewer chunks at B*H < 32 (the state recurrence alone, KDA gate, graph replay, us,
# direct / segmented / affine-step): B*H = 24 96 chunks 197 / 180 / 225, 192 chunks 401 / 338 /
# 443, 64 chunks 114 / 134 / 149; B*H = 16 96 chunks 157 / 136 / 166, 192 chunks 375 / 229 / 350,
# 64 chunks 108 / 113 / 104; B*H = 8 128 chunks 203 / 128 / 138, 96 chunks 155 / 117 / 102;
# B*H = 4 192 chunks 303 / 141 / 160, 128 chunks 204 / 118 / 110; B*H = 32 128 chunks
# 273 / 286 / 362, 192 chunks 412 / 414 / 546
SEG_SHORT_MAX_BH = 32
SEG_SHORT_MIN_CHUNKS = 96           # B*H >= 16
SEG_NARROW_MIN_CHUNKS = 128         # B*H < 16, with B*H*NT >= SEG_NARROW_MIN_WORK
SEG_NARROW_MIN_WORK = 768


def segments_for(B, H, NT):
    """Segment count of the segmented form for B rows of NT chunks and H heads."""
    s = max(1, SEG_TARGET_GROUPS // (4 * B * H))
    return max(1, min(s, NT // SEG_MIN_LEN))


def _state_method(method, B, H, NT):
    """Which form of the backward state recurrence runs: direct, affine or segmented."""
    if method not in ("auto", "direct", "affine", "segmented"):
        raise ValueError('method must be "auto", "direct", "affine" or "segmented"')
    if method != "auto":
        return method
    if NT >= SEG_MIN_CHUNKS and B * H < SEG_MAX_BH:
        return "segmented"
    if B * H < SEG_SHORT_MAX_BH and (NT >= SEG_SHORT_MIN_CHUNKS if B * H >= 16 else
                                     NT >= SEG_NARROW_MIN_CHUNKS and B * H * NT >= SEG_NARROW_MIN_WORK):
        return "segmented"
    if B * H <= AFFINE_MAX_BH and NT >= AFFINE_STATE_MIN_CHUNKS:
        return "affine"
    return "direct"


# Recompute policy: the forward scan (direct) and the backward state recurrence are
# independent.  With few heads and long rows the scan runs beside the segmented recurrence
# (each leaves most of the GPU idle), in place of the affine-step pair or the direct
# kernels one after the other; a packed batch that the fused sweep (fwd_h_wy_pays) does
# not take runs the scan beside the direct recurrence (its short sequences leave CUs idle
# while the longest one runs).  SIDE_BY_SIDE switches both off.
SIDE_BY_SIDE = True
SBS_MIN_BH = 8
SBS_MIN_WORK = 1024       # B * H * NT


def side_by_side_pays(B, H, NT):
    """True when the recompute policy runs the forward scan beside the segmented state
    recurrence for B rows of NT chunks and H heads (dense rows).  Measured crossovers
    (DeltaNet / GDN): it beats the affine-step pair from B*H*NT = 1024 at B*H >= 8 (B*H = 16,
    NT = 128: 405 vs 503 us) but not at B*H = 4 (NT = 128: 205 vs 160 us); with more heads
    the direct kernels win until the segmented form's own threshold."""
    BH = B * H
    if not SIDE_BY_SIDE or BH < SBS_MIN_BH or 2 * BH >= 256 or BH * NT < SBS_MIN_WORK:
        return False
    return BH <= AFFINE_MAX_BH or NT >= SEG_MIN_CHUNKS


# Paired direct recurrences (recompute policy): when batch x heads is too small for one
# direct recurrence to fill the GPU, the forward scan and the backward state recurrence run
# side by side at a common value-tile width chosen so that the two launches together hold
# at most one work-group per CU.
PAIRED = True
PAIRED_MIN_BH = 17
# ... at 64-wide tiles up to this many work-groups per launch: while one recurrence alone
# leaves CUs idle the pair still wins, the second launch's work-groups taking the CUs the first
# leaves (B*H = 72-124: 12-26 % faster); at B*H = 128 each fills the GPU (5 % slower paired)
PAIRED_MAX_GROUPS = 254
# ... and at 16-wide tiles for B*H <= 16 (at most 128 work-groups each) on short rows, where
# the pair (one launch) beats the affine-step form and the direct recurrences one after the
# other: rows of at most 8 chunks at any such B*H, of at most 128 from B*H = 12
PAIRED16_SHORT_NT = 8
PAIRED16_MID_BH = 12
PAIRED16_MID_NT = 128
# ... as one launch (fdr_paired_recurrences) instead of two kernels on two streams joined by
# events, whose fork and join cost ~25 us of host time per backward
PAIRED_ONE_LAUNCH = True
# ... and, scalar / no gate at value tiles up to this width, Aqk written by fdr_prepare_wu and
# read by the state recurrence instead of formed there: at narrow tiles every one of a head's
# value-tile work-groups would form the whole Aqk again on its step chain (GDN B=1 T=2048 H=16
# 100.5 vs 113.5 us, B=2 T=2048 H=16 146.0 vs 153.4, B=1 T=6144 H=16 296 vs 339, DeltaNet B=1
# T=2048 H=16 92.1 vs 97.7; at 64-wide tiles, GDN B=4 T=2048 H=16, 271.3 vs 268.4)
PAIRED_AQK_MAX_VB = 32
# ... with u formed inside the scan (fwd_h_u) instead of written by prepare_wu and read back
PAIRED_U = True
# ... and, for GDN / DeltaNet, prepare + paired recurrences + chunk stage as one library call
# (fdr_scalar_bwd: the same launches and bits, one workspace allocation for the intermediates)
SCALAR_ONE_CALL = True
# ... and, vector gates at 64-wide tiles, with qg / kg formed from the raw q / k where each
# recurrence stages a chunk (fdr_state_bwd_raw_qk, fwd_h_u) instead of written by prepare_wu and
# read back.  (At 32-wide tiles every one of a head's four value tiles would form them again:
# measured slower there.)
PAIRED_RAW = True
# ... and, GDN2 (a vector b) at 64-wide tiles, w formed in both recurrences too (w = Akk (b k 2^g)
# from the same staged k and gate tile), so that fdr_prepare_wu does not run at all.  (KDA's
# prepare, with a scalar beta, and GDN2's at B*H = 32 cost less than forming w adds to the state
# recurrence's step: not taken there.)
PAIRED_FORMW = True


def paired_tile(B, H, NT, gate_mode):
    """Value-tile width at which the recompute policy runs ``fwd_h`` and ``state_bwd`` (both
    direct) side by side, or 0 when it runs them otherwise: 32-wide tiles for 17 <= B H <= 32
    (at most 128 work-groups each, the two together one per CU), 64-wide ones up to B H = 127
    (``PAIRED_MAX_GROUPS``), and for B H <= 16 16-wide tiles on short rows (``PAIRED16_*``).
    Measured (MI355X):
    GDN2 B=2 T=8192 H=32 both recurrences 0.451 ms paired at
    64-wide tiles vs 0.544 one after the other at 32-wide; B=2 T=4096 H=16 0.177 (32-wide) vs
    0.231; B=1 T=8192 H=48 0.443 vs 0.543; B=1 T=16384 H=24 0.639 (32-wide) vs 0.905.  The
    scalar / no-gate families, whose fused sweep (``fwd_h_wy_pays``) runs from B H = 64: GDN
    B=4 T=2048 H=16 backward 0.288 ms paired (64-wide, u formed in the scan) vs 0.311 with the
    sweep, DeltaNet same shape 0.261 vs 0.279; DeltaNet B=2 T=2048 H=16 (graph replay)
    148.6 us paired (32-wide) vs 178.4 us.  At B H = 16 against the affine-step form (graph
    replay, backward): B=1 T=2048 H=16 DeltaNet 97 vs 112 us, GDN 113 vs 117, KDA 112 vs 129,
    GDN2 122 vs 138; T=4096 DeltaNet 179 vs 199, KDA 226 vs 236 (GDN, GDN2 within 1.5 %);
    T=8192 GDN 447 vs 421.  As one launch (``PAIRED_ONE_LAUNCH``), graph
    replay: rows of 4-8 chunks at B H = 1-8 DeltaNet 25.5-37.0 vs 30.3-46.0 us, KDA 31.1-38.8 vs
    35.3-50.6 (configs[0], B=1 T=256 H=2: DeltaNet 30.0 vs 36.7); 16 chunks at B H = 12 DeltaNet
    55.5 vs 57.5, 32 chunks KDA 102.5 vs 107.6; but 16-24 chunks at B H = 2-8 DeltaNet 50.7-67.2 vs
    46.4-61.6 and 32 chunks at B H = 4-8 72-83 vs 61-72 (the affine-step form's cheaper steps).
    At B H = 16 against the scan beside the segmented recurrence: 96 chunks DeltaNet 282 vs 323 us,
    GDN 333 vs 343, KDA 340 vs 376, GDN2 378 vs 408; 128 chunks (GDN / DeltaNet reading Aqk)
    DeltaNet 379 vs 389, GDN 409 vs 419, KDA 457 vs 473, GDN2 518 vs 511 (eager all 3-9 % faster);
    B H = 12, 64 chunks: DeltaNet 160 vs 204, KDA 187 vs 206; 128 chunks: GDN 358 vs 379, KDA 399 vs
    408.  B H = 17-23 at 32-wide tiles, against the recurrences one after the other: B=1 T=2048
    H=20 DeltaNet 118 vs 156 us, GDN 129 vs 179, KDA 136 vs 171, GDN2 153 vs 189; KDA T=4096 H=18
    259 vs 320.  B H = 65-127 at 64-wide tiles (up to 254 work-groups a launch), against the fused
    sweep or the recurrences one after the other: B=1 T=2048 H=72 DeltaNet 327 vs 444 us, H=96 GDN
    432 vs 555, H=112 KDA 570 vs 650, H=120 GDN2 645 vs 779, H=124 DeltaNet 464 vs 558; at B H = 128
    (256 work-groups each) GDN B=8 T=4096 H=16 975 vs 928, KDA B=1 T=4096 H=128 1179 vs 1114."""
    BH = B * H
    if not PAIRED or NT < 1:
        return 0
    if BH >= PAIRED_MIN_BH:
        if BH * (V_SUPPORTED // 32) <= 128:
            return 32
        if BH * (V_SUPPORTED // 64) <= PAIRED_MAX_GROUPS:
            return 64
        return 0
    if BH * (V_SUPPORTED // 16) <= 128 and (NT <= PAIRED16_SHORT_NT or (BH >= PAIRED16_MID_BH and NT <= PAIRED16_MID_NT)):
        return 16
    return 0


def state_form(B, H, NT):
    """The form ``state_bwd(method="auto")`` takes for B rows of NT chunks and H heads."""
    return _state_method("auto", B, H, NT)


def _use_affine(method, B, H, NT):
    if method not in ("auto", "direct", "affine"):
        raise ValueError('method must be "auto", "direct" or "affine"')
    if method == "auto":
        return B * H <= AFFINE_MAX_BH and NT >= AFFINE_MIN_CHUNKS
    return method == "affine"


def affine_pays(x):
    """True when the affine-step recurrences are the faster choice for the shape of x,
    a [B, T, H, .] tensor with one head per state (value heads), for the recompute policy
    (both recurrences)."""
    B, T, H = x.shape[:3]
    return _use_affine("auto", B, H, T // CHUNK) and not side_by_side_pays(B, H, T // CHUNK)


def _affine_workspace(B, NT, H, dev):
    """Step matrices (bf16 K x K) and offsets (fp32 K x V) of every chunk-head."""
    n = B * NT * H
    return (torch.empty(n, K_SUPPORTED, K_SUPPORTED, device=dev, dtype=torch.bfloat16),
            torch.empty(n, K_SUPPORTED, V_SUPPORTED, device=dev, dtype=torch.float32))


def _chunk_offsets(chunk_offsets, B, T, dev):
    """Validated (int32 device tensor, N) for a packed variable-length batch, or (None, B).

    chunk_offsets[n] is the first chunk of sequence n (FLA's prepare_chunk_offsets over
    chunk-aligned cu_seqlens): starts at 0, ends at T / 64, never decreases (an empty
    sequence passes its state through: dh0 = dht, final = h0)."""
    if chunk_offsets is None:
        return None, B
    if B != 1:
        raise ValueError("a variable-length batch is packed along T: B must be 1")
    co = torch.as_tensor(chunk_offsets)
    host = co.detach().to("cpu", torch.int64)
    if host.ndim != 1 or host.numel() < 2:
        raise ValueError("chunk_offsets must be [N+1] with N >= 1")
    if int(host[0]) != 0 or int(host[-1]) != T // CHUNK or bool((host[1:] < host[:-1]).any()):
        raise ValueError(f"chunk_offsets must rise from 0 to T/{CHUNK} = {T // CHUNK}")
    return co.to(device=dev, dtype=torch.int32).contiguous(), host.numel() - 1


class Varlen:
    """A packed variable-length batch (B = 1): FLA's ``cu_seqlens`` [N+1] and what the kernels
    take with it, on the device -- ``chunk_indices`` [NC, 2] (sequence, chunk of the sequence;
    FLA prepare_chunk_indices) and ``chunk_offsets`` [N+1] (FLA prepare_chunk_offsets), each
    sequence cut into ceil(len / 64) chunks.  Sequences start anywhere; when every one starts
    on a 64-token boundary and T is a multiple of 64 (``aligned``) the dense kernels serve the
    chunk-local stages and only the scans take the offsets."""

    def __init__(self, cu_seqlens, device):
        host = torch.as_tensor(cu_seqlens).detach().to("cpu", torch.int64)
        if host.ndim != 1 or host.numel() < 2 or int(host[0]) != 0:
            raise ValueError("cu_seqlens must be [N+1], starting at 0")
        lens = host[1:] - host[:-1]
        if bool((lens < 0).any()):
            raise ValueError("cu_seqlens must not decrease")
        nch = (lens + CHUNK - 1) // CHUNK
        self.N = int(lens.numel())
        self.T = int(host[-1])
        self.NC = int(nch.sum())
        self.max_chunks = int(nch.max())
        if self.NC == 0:
            raise ValueError("a variable-length batch needs at least one token")
        self.aligned = bool((host % CHUNK == 0).all())
        seq = torch.repeat_interleave(torch.arange(self.N), nch)
        first = torch.cumsum(nch, 0) - nch
        ci = torch.stack([seq, torch.arange(self.NC) - first[seq]], 1)
        i32 = dict(device=device, dtype=torch.int32)
        self.cu_seqlens = host.to(**i32)
        self.chunk_indices = ci.to(**i32).contiguous()
        self.chunk_offsets = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(nch, 0)]).to(**i32)

    def check(self, x):
        if x.shape[0] != 1 or x.shape[1] != self.T:
            raise ValueError(f"a variable-length batch is [1, {self.T}, ...], got {tuple(x.shape)}")


def _rows(x, varlen):
    """(B, T, H, K) of a token-major operand; T any length for a packed variable-length batch."""
    if varlen is None:
        return _dims(x)
    if x.ndim != 4:
        raise ValueError("q must be [B,T,H,K]")
    varlen.check(x)
    if x.shape[3] != K_SUPPORTED:
        raise ValueError(f"K must be {K_SUPPORTED}")
    if x.device.type != "cuda":
        raise ValueError("HIP backward requires a GPU tensor")
    return x.shape


def _mapped(varlen):
    """The variable-length batch when the chunk-local kernels need its row map, else None."""
    return None if varlen is None or varlen.aligned else varlen


def _group(H, HQ):
    """Value heads H and q / k heads HQ (grouped value heads: H a multiple of HQ)."""
    if HQ <= 0 or H % HQ:
        raise ValueError(f"value heads ({H}) must be a multiple of the q/k heads ({HQ})")
    return H, HQ


def _dims(q):
    if q.ndim != 4:
        raise ValueError("q must be [B,T,H,K]")
    B, T, H, K = q.shape
    if K != K_SUPPORTED:
        raise ValueError(f"K must be {K_SUPPORTED}")
    if T <= 0 or T % CHUNK:
        raise ValueError(f"T must be a positive multiple of {CHUNK}")
    if q.device.type != "cuda":
        raise ValueError("HIP backward requires a GPU tensor")
    return B, T, H, K


def state_bwd(q, k, w, g, gate_mode, dO, scale, aqk=None, dv=None, dht=None, want_dh0=True,
              value_block=0, method="auto", chunk_offsets=None, segments=0, state_v_first=False, varlen=None,
              raw_qk=False, beta=None, b=None, Akk=None):
    """Reverse state recurrence.  Returns (dh [B,NT,H,K,V] bf16, dR [B,T,H,V] bf16, dh0 fp32|None).

    dv_local = Aqk^T dO comes from ``aqk``, or is given as ``dv``; with neither (scalar / no
    gate, direct form), Aqk = scale tril(q k^T 2^(g_i - g_s)) is formed in-kernel from the raw
    q / k the recurrence stages anyway.

    ``chunk_offsets`` (int [N+1]): B = 1 holds N sequences packed along T, sequence n on
    chunks [chunk_offsets[n], chunk_offsets[n+1]); dht / dh0 are then [N,H,K,V] and the
    direct kernel runs (fdr_state_bwd_varlen).  ``varlen`` (a ``Varlen``): the same for
    sequences starting anywhere (dh then has ``varlen.NC`` chunks).  ``state_v_first``: dht and dh0 are [.., V, K]
    (FLA's layout); the per-chunk dh is [B,NT,H,K,V] either way.

    method "direct": one kernel (fdr_state_bwd); "affine": chunk-parallel step
    matrices, a one-product-per-chunk scan and a chunk-parallel dR pass
    (fdr_affine_*), faster when B*H is too small to fill the GPU; "segmented": every row
    split into ``segments`` (0: ``segments_for``) whose affine maps are formed in parallel,
    chained, and each segment rerun from its end state (fdr_state_bwd_segmented), for long
    rows and few heads; "auto" picks.

    ``raw_qk`` (vector gate, ``aqk``, dense rows, direct form): q and k are the raw ones and
    qg = q 2^g, kg = k 2^(g_last - g) are formed in-kernel with ``prepare_wu``'s roundings
    (fdr_state_bwd_raw_qk), so the result is the bits of ``prepare_wu``'s qg / kg then this.
    With ``raw_qk``, w may be None: then w = Akk (beta k 2^g), or Akk (b k 2^g) for GDN2, is
    formed in-kernel as ``prepare_wu`` forms it (``Akk`` and one of ``beta`` / ``b``)."""
    B, T, HQ, K = _rows(q, varlen)
    H, HQ = _group(w.shape[2] if w is not None and w.ndim == 4 else dO.shape[2], HQ)
    V = V_SUPPORTED
    dev = q.device
    bf, f32 = torch.bfloat16, torch.float32
    for x, n in ((q, "q"), (k, "k")):
        _need(x, n, bf, (B, T, HQ, K), dev)
    if w is not None:
        _need(w, "w", bf, (B, T, H, K), dev)
    else:
        if not raw_qk:
            raise ValueError("w is formed in-kernel only with raw_qk")
        _need(Akk, "Akk", f32, (B, T, H, CHUNK), dev)
        if (beta is None) == (b is None):
            raise ValueError("w formed in-kernel: pass exactly one of beta / b")
        if b is not None:
            _need(b, "b", bf, (B, T, H, K), dev)
        else:
            _need(beta, "beta", f32, (B, T, H), dev)
    _need(dO, "dO", bf, (B, T, H, V), dev)
    if gate_mode == GATE_VECTOR:
        _need(g, "g", f32, (B, T, H, K), dev)
    elif gate_mode == GATE_SCALAR:
        _need(g, "g", f32, (B, T, H), dev)
    elif gate_mode != GATE_NONE:
        raise ValueError("gate_mode must be 0, 1 or 2")
    inline = aqk is None and dv is None
    if aqk is not None and dv is not None:
        raise ValueError("pass at most one of aqk / dv")
    if inline and gate_mode == GATE_VECTOR:
        raise ValueError("Aqk is formed in-kernel for the scalar / no-gate families only: pass aqk")
    if aqk is not None:
        _need(aqk, "Aqk", f32, (B, T, H, CHUNK), dev)
    if dv is not None:
        _need(dv, "dv", bf, (B, T, H, V), dev)
    if varlen is not None:
        if chunk_offsets is not None:
            raise ValueError("pass chunk_offsets or varlen, not both")
        co, N, NT = varlen.chunk_offsets, varlen.N, varlen.NC
    else:
        co, N = _chunk_offsets(chunk_offsets, B, T, dev)
        NT = T // CHUNK
    if dht is not None:
        _need(dht, "dht", f32, (N, H, K, V), dev)
    if value_block not in (0, 16, 32, 64):
        raise ValueError("value_block must be 0, 16, 32 or 64")
    vf = int(bool(state_v_first))
    dh = torch.empty(B, NT, H, K, V, device=dev, dtype=bf)
    dr = torch.empty(B, T, H, V, device=dev, dtype=bf)
    dh0 = torch.empty(N, H, K, V, device=dev, dtype=f32) if want_dh0 else None
    P = _lib.ptr
    if raw_qk:
        if gate_mode != GATE_VECTOR or aqk is None or co is not None or method not in ("auto", "direct"):
            raise ValueError("raw_qk takes a vector gate, aqk, dense rows and the direct form")
        formw = w is None
        st = _lib.load().fdr_state_bwd_raw_qk(P(q), P(k), P(w), P(g), P(beta if formw else None),
                                              P(b if formw else None), P(Akk if formw else None), P(dO), P(aqk),
                                              P(dht), P(dh), P(dr), P(dh0), vf, B, T, H, HQ, K, V, CHUNK,
                                              float(scale), int(value_block), _lib.stream_handle(dev))
        _lib.check(st, "fdr_state_bwd_raw_qk")
        return dh, dr, dh0
    if co is not None:
        if method == "affine":
            raise ValueError("the affine-step form takes equal-length rows, not chunk_offsets")
        cu = _mapped(varlen)
        st = _lib.load().fdr_state_bwd_varlen(P(q), P(k), P(w), P(g), int(gate_mode), P(dO), P(aqk), P(dv),
                                              P(dht), P(dh), P(dr), P(dh0), vf, P(co),
                                              None if cu is None else P(cu.cu_seqlens), N, NT, H, HQ, K, V,
                                              CHUNK, float(scale), int(value_block), _lib.stream_handle(dev))
        _lib.check(st, "fdr_state_bwd_varlen")
        return dh, dr, dh0
    form = _state_method(method, B, H, NT)
    if (HQ != H or inline) and form != "direct":
        if method != "auto":
            raise ValueError("grouped q/k heads and the in-kernel Aqk take the direct state recurrence")
        form = "direct"
    if form == "segmented":
        segs = int(segments) or segments_for(B, H, NT)
        if not 1 <= segs <= NT:
            raise ValueError(f"segments must be in [1, {NT}]")
        lib = _lib.load()
        ws = torch.empty(lib.fdr_state_bwd_segmented_workspace_bytes(B, H, segs) // 4, device=dev, dtype=f32)
        st = lib.fdr_state_bwd_segmented(P(q), P(k), P(w), P(g), int(gate_mode), P(dO), P(aqk), P(dv), P(dht),
                                         P(dh), P(dr), P(dh0), vf, B, T, H, K, V, CHUNK, float(scale), segs,
                                         int(value_block), P(ws), _lib.stream_handle(dev))
        _lib.check(st, "fdr_state_bwd_segmented")
        return dh, dr, dh0
    if form == "affine":
        vb = value_block or AFFINE_VALUE_BLOCK
        step, offset = _affine_workspace(B, NT, H, dev)
        dv_local = torch.empty(B, T, H, V, device=dev, dtype=bf) if aqk is not None else None
        lib = _lib.load()
        st = lib.fdr_affine_prep_bwd(P(q), P(k), P(w), P(g), int(gate_mode), P(dO), P(aqk), P(dv), P(step),
                                     P(offset), P(dv_local), B, T, H, K, V, CHUNK, float(scale),
                                     _lib.stream_handle(dev))
        _lib.check(st, "fdr_affine_prep_bwd")
        arr, n = _lib.problems(_lib.ScanProblem, [_lib.ScanProblem(
            P(step), P(offset), P(g), P(dht), P(dh), P(dh0), int(gate_mode), 1, vf)])
        _lib.check(lib.fdr_affine_scan(arr, n, B, T, H, K, V, CHUNK, int(vb), _lib.stream_handle(dev)),
                   "fdr_affine_scan")
        arr, n = _lib.problems(_lib.SideProblem, [_lib.SideProblem(
            P(k), P(dh), P(dv_local if dv is None else dv), P(g) if gate_mode == GATE_SCALAR else None,
            P(dr), 1.0)])
        _lib.check(lib.fdr_affine_side(arr, n, B, T, H, K, V, CHUNK, _lib.stream_handle(dev)), "fdr_affine_side")
        return dh, dr, dh0
    st = _lib.load().fdr_state_bwd(P(q), P(k), P(w), P(g), int(gate_mode), P(dO), P(aqk), P(dv),
                                   P(dht), P(dh), P(dr), P(dh0), vf, B, T, H, HQ, K, V, CHUNK,
                                   float(scale), int(value_block), _lib.stream_handle(dev))
    _lib.check(st, "fdr_state_bwd")
    return dh, dr, dh0


def recurrences(q, k, w, u, g, gate_mode, dO, scale, aqk=None, dv=None, h0=None, dht=None, want_dh0=True,
                value_block=0, state_v_first=False):
    """Both state recurrences of the recompute policy in one pass of the affine-step
    kernels, the forward and the backward recurrence side by side (neither needs the
    other's states).  q/k as for ``state_bwd`` (qg/kg for a vector gate); w, u from
    ``prepare_wu``.  Returns (h, v_new, dh, dR, dh0|None), each as ``fwd_h`` /
    ``state_bwd`` return them."""
    B, T, H, K = _dims(q)
    V = V_SUPPORTED
    dev = q.device
    bf, f32 = torch.bfloat16, torch.float32
    for x, n in ((q, "q"), (k, "k"), (w, "w")):
        _need(x, n, bf, (B, T, H, K), dev)
    _need(u, "u", bf, (B, T, H, V), dev)
    _need(dO, "dO", bf, (B, T, H, V), dev)
    if gate_mode == GATE_VECTOR:
        _need(g, "g", f32, (B, T, H, K), dev)
    elif gate_mode == GATE_SCALAR:
        _need(g, "g", f32, (B, T, H), dev)
    elif gate_mode != GATE_NONE:
        raise ValueError("gate_mode must be 0, 1 or 2")
    if (aqk is None) == (dv is None):
        raise ValueError("exactly one of aqk / dv is required")
    if aqk is not None:
        _need(aqk, "Aqk", f32, (B, T, H, CHUNK), dev)
    if dv is not None:
        _need(dv, "dv", bf, (B, T, H, V), dev)
    for x, n in ((h0, "h0"), (dht, "dht")):
        if x is not None:
            _need(x, n, f32, (B, H, K, V), dev)
    if value_block not in (0, 16, 32, 64):
        raise ValueError("value_block must be 0, 16, 32 or 64")
    vb = value_block or AFFINE_VALUE_BLOCK
    NT = T // CHUNK
    h = torch.empty(B, NT, H, K, V, device=dev, dtype=bf)
    vnew = torch.empty(B, T, H, V, device=dev, dtype=bf)
    dh = torch.empty(B, NT, H, K, V, device=dev, dtype=bf)
    dr = torch.empty(B, T, H, V, device=dev, dtype=bf)
    dh0 = torch.empty(B, H, K, V, device=dev, dtype=f32) if want_dh0 else None
    sb, ob = _affine_workspace(B, NT, H, dev)
    sf, of = _affine_workspace(B, NT, H, dev)
    dv_local = torch.empty(B, T, H, V, device=dev, dtype=bf) if aqk is not None else None
    P = _lib.ptr
    lib = _lib.load()
    stream = _lib.stream_handle(dev)
    _lib.check(lib.fdr_affine_prep_pair(P(q), P(k), P(w), P(u), P(g), int(gate_mode), P(dO), P(aqk), P(dv),
                                        P(sb), P(ob), P(dv_local), P(sf), P(of), B, T, H, K, V, CHUNK,
                                        float(scale), stream), "fdr_affine_prep_pair")
    arr, n = _lib.problems(_lib.ScanProblem, [
        _lib.ScanProblem(P(sb), P(ob), P(g), P(dht), P(dh), P(dh0), int(gate_mode), 1, int(bool(state_v_first))),
        _lib.ScanProblem(P(sf), P(of), P(g), P(h0), P(h), None, int(gate_mode), 0, int(bool(state_v_first)))])
    _lib.check(lib.fdr_affine_scan(arr, n, B, T, H, K, V, CHUNK, int(vb), stream), "fdr_affine_scan")
    arr, n = _lib.problems(_lib.SideProblem, [
        _lib.SideProblem(P(k), P(dh), P(dv_local if dv is None else dv),
                         P(g) if gate_mode == GATE_SCALAR else None, P(dr), 1.0),
        _lib.SideProblem(P(w), P(h), P(u), None, P(vnew), -1.0)])
    _lib.check(lib.fdr_affine_side(arr, n, B, T, H, K, V, CHUNK, stream), "fdr_affine_side")
    return h, vnew, dh, dr, dh0


def chunk_bwd(q, k, v, v_new, dO, dR, g, gate_mode, Akk, h, dh, scale, beta=None, b=None, w=None,
              gate_fold=None, beta_sigmoid=0.0, h_v_first=False, varlen=None):
    """Fused residual-WY + matrix-intra + epilogue stage.

    ``gate_fold`` (KDA only) = dict(g_raw, A_log, dt_bias, lower_bound): the in-kernel gate's
    backward is applied where dg is formed; ``dg`` is then dL/dg_raw (g_raw's dtype) and the
    result also holds ``dA_log`` / ``ddt_bias`` (fp32, or None).

    ``beta_sigmoid`` = s > 0 (scalar beta): beta was activated as s * sigmoid(x) in the
    forward, and ``dbeta`` is returned as dL/dx (the reference's fused beta-sigmoid backward).
    ``h_v_first`` (vector gates): the saved per-chunk states ``h`` are [B,NT,H,V,K].
    ``varlen`` (a ``Varlen``): a packed variable-length batch; h, dh have ``varlen.NC`` chunks.

    Returns dict(dq, dk, dv [bf16], dg [fp32, gate shape] | None, dbeta [fp32] | None,
    db, dw [bf16] | None)."""
    B, T, HQ, K = _rows(q, varlen)
    H, HQ = _group(v.shape[2] if v is not None and v.ndim == 4 else HQ, HQ)
    V = V_SUPPORTED
    dev = q.device
    bf, f32 = torch.bfloat16, torch.float32
    NT = T // CHUNK if varlen is None else varlen.NC
    mv = _mapped(varlen)
    for x, n in ((q, "q"), (k, "k")):
        _need(x, n, bf, (B, T, HQ, K), dev)
    for x, n in ((v, "v"), (v_new, "v_new"), (dO, "dO"), (dR, "dR")):
        _need(x, n, bf, (B, T, H, V), dev)
    _need(Akk, "Akk", f32, (B, T, H, CHUNK), dev)
    _need(h, "h", bf, (B, NT, H, K, V), dev)
    _need(dh, "dh", bf, (B, NT, H, K, V), dev)
    vec_b = b is not None
    if vec_b:
        if gate_mode != GATE_VECTOR:
            raise ValueError("vector erase/write gates require a vector decay gate")
        _need(b, "b", bf, (B, T, H, K), dev)
        _need(w, "w", bf, (B, T, H, V), dev)
    else:
        _need(beta, "beta", f32, (B, T, H), dev)
    if gate_mode == GATE_VECTOR:
        _need(g, "g", f32, (B, T, H, K), dev)
    elif gate_mode == GATE_SCALAR:
        _need(g, "g", f32, (B, T, H), dev)
    elif gate_mode != GATE_NONE:
        raise ValueError("gate_mode must be 0, 1 or 2")
    beta_sigmoid = float(beta_sigmoid or 0.0)
    if beta_sigmoid < 0 or (beta_sigmoid and vec_b):
        raise ValueError("beta_sigmoid is a non-negative scale of a scalar beta")
    hvf = int(bool(h_v_first))
    if hvf and gate_mode != GATE_VECTOR:
        raise ValueError("[V,K] saved states come with the vector-gate families")
    if gate_fold is not None:
        return _chunk_bwd_gate_fold(q, k, v, v_new, dO, dR, g, gate_mode, Akk, h, dh, scale, beta, b, gate_fold,
                                    beta_sigmoid, hvf, H, mv)
    out = dict(dq=torch.empty(B, T, H, K, device=dev, dtype=bf),
               dk=torch.empty(B, T, H, K, device=dev, dtype=bf),
               dv=torch.empty(B, T, H, V, device=dev, dtype=bf),
               dg=torch.empty_like(g) if gate_mode != GATE_NONE else None,
               dbeta=None if vec_b else torch.empty(B, T, H, device=dev, dtype=f32),
               db=torch.empty(B, T, H, K, device=dev, dtype=bf) if vec_b else None,
               dw=torch.empty(B, T, H, V, device=dev, dtype=bf) if vec_b else None)
    P = _lib.ptr
    common = (P(q), P(k), P(v), P(v_new), P(dO), P(dR), P(g), int(gate_mode), P(beta), P(b), P(w), P(Akk), P(h),
              P(dh), P(out["dq"]), P(out["dk"]), P(out["dv"]), P(out["dg"]), P(out["dbeta"]), beta_sigmoid,
              P(out["db"]), P(out["dw"]), hvf)
    if mv is not None:
        st = _lib.load().fdr_chunk_bwd_varlen(*common, P(mv.cu_seqlens), P(mv.chunk_indices), mv.NC, H, HQ, K, V,
                                              CHUNK, float(scale), _lib.stream_handle(dev))
        _lib.check(st, "fdr_chunk_bwd_varlen")
        return out
    st = _lib.load().fdr_chunk_bwd(*common, B, T, H, HQ, K, V, CHUNK, float(scale), _lib.stream_handle(dev))
    _lib.check(st, "fdr_chunk_bwd")
    return out


def chunk_bwd_wy(q, k, v, v_new, dO, dR, g, Akk, h, dh, scale, beta=None, h_v_first=False, b=None, w=None,
                 varlen=None):
    """The WY seam alone: every term of ``chunk_bwd`` but the matrix intra.  KDA (``beta``,
    fdr_chunk_bwd_wy) returns dict(dq, dk [fp32], dv [bf16], dbeta [fp32, complete on
    |beta| >= 1e-6 rows], dg [fp32, before the in-chunk reverse cumsum], dA [fp32
    [B,T,H,64], the intra's dAkk]); GDN2 (``b``, ``w``: erase and write gates,
    fdr_gdn2_chunk_bwd_wy) returns dict(dq, dk, dv, db [fp32, without the intra's ue k],
    dw [bf16], dg, dA).  ``varlen``: a packed variable-length batch (``Varlen``; h, dh then
    have ``varlen.NC`` chunks)."""
    B, T, HQ, K = _rows(q, varlen)
    H, HQ = _group(v.shape[2] if v is not None and v.ndim == 4 else HQ, HQ)
    V = V_SUPPORTED
    dev = q.device
    bf, f32 = torch.bfloat16, torch.float32
    NT = T // CHUNK if varlen is None else varlen.NC
    if varlen is None and T % CHUNK:
        raise ValueError("T must be a multiple of 64 (pass cu_seqlens for ragged rows)")
    for x, n in ((q, "q"), (k, "k")):
        _need(x, n, bf, (B, T, HQ, K), dev)
    for x, n in ((v, "v"), (v_new, "v_new"), (dO, "dO"), (dR, "dR")):
        _need(x, n, bf, (B, T, H, V), dev)
    _need(g, "g", f32, (B, T, H, K), dev)
    vec_b = b is not None
    if vec_b == (beta is not None):
        raise ValueError("exactly one of beta (KDA) / b, w (GDN2) is required")
    if vec_b:
        if HQ != H:
            raise ValueError("GDN2 takes one q/k head per value head")
        _need(b, "b", bf, (B, T, H, K), dev)
        _need(w, "w", bf, (B, T, H, V), dev)
    else:
        _need(beta, "beta", f32, (B, T, H), dev)
    _need(Akk, "Akk", f32, (B, T, H, CHUNK), dev)
    _need(h, "h", bf, (B, NT, H, V, K) if h_v_first else (B, NT, H, K, V), dev)
    _need(dh, "dh", bf, (B, NT, H, K, V), dev)
    out = dict(dq=torch.empty(B, T, H, K, device=dev, dtype=f32), dk=torch.empty(B, T, H, K, device=dev, dtype=f32),
               dv=torch.empty(B, T, H, V, device=dev, dtype=bf), dg=torch.empty(B, T, H, K, device=dev, dtype=f32),
               dA=torch.empty(B, T, H, CHUNK, device=dev, dtype=f32))
    if vec_b:
        out["db"] = torch.empty(B, T, H, K, device=dev, dtype=f32)
        out["dw"] = torch.empty(B, T, H, V, device=dev, dtype=bf)
    else:
        out["dbeta"] = torch.empty(B, T, H, device=dev, dtype=f32)
    P = _lib.ptr
    lib = _lib.load()
    hv = int(bool(h_v_first))
    head = (P(q), P(k), P(v), P(v_new), P(dO), P(dR), P(g))
    mv = _mapped(varlen)
    if vec_b:
        tail = (P(Akk), P(h), P(dh), P(out["dq"]), P(out["dk"]), P(out["dv"]), P(out["db"]), P(out["dw"]),
                P(out["dg"]), P(out["dA"]), hv)
        if mv is not None:
            st = lib.fdr_gdn2_chunk_bwd_wy_varlen(*head, P(b), P(w), *tail, P(mv.cu_seqlens), P(mv.chunk_indices),
                                                  mv.NC, H, K, V, CHUNK, float(scale), _lib.stream_handle(dev))
        else:
            st = lib.fdr_gdn2_chunk_bwd_wy(*head, P(b), P(w), *tail, B, T, H, K, V, CHUNK, float(scale),
                                           _lib.stream_handle(dev))
        _lib.check(st, "fdr_gdn2_chunk_bwd_wy")
        return out
    tail = (P(Akk), P(h), P(dh), P(out["dq"]), P(out["dk"]), P(out["dv"]), P(out["dbeta"]), P(out["dg"]),
            P(out["dA"]), hv)
    if mv is not None:
        st = lib.fdr_chunk_bwd_wy_varlen(*head, P(beta), *tail, P(mv.cu_seqlens), P(mv.chunk_indices), mv.NC, H,
                                         HQ, K, V, CHUNK, float(scale), _lib.stream_handle(dev))
    else:
        st = lib.fdr_chunk_bwd_wy(*head, P(beta), *tail, B, T, H, HQ, K, V, CHUNK, float(scale),
                                  _lib.stream_handle(dev))
    _lib.check(st, "fdr_chunk_bwd_wy")
    return out


def chunk_bwd_original(q, k, v, v_new, dO, dR, g, Akk, h, dh, scale, beta):
    """KDA's chunk stage in the original 7-product formulation (fdr_chunk_bwd_original): the
    same-GPU comparator of ``chunk_bwd``.  Returns dict(dq, dk, dv, dg, dbeta)."""
    B, T, H, K = _dims(q)
    V = V_SUPPORTED
    dev = q.device
    bf, f32 = torch.bfloat16, torch.float32
    NT = T // CHUNK
    for x, n in ((q, "q"), (k, "k")):
        _need(x, n, bf, (B, T, H, K), dev)
    for x, n in ((v, "v"), (v_new, "v_new"), (dO, "dO"), (dR, "dR")):
        _need(x, n, bf, (B, T, H, V), dev)
    _need(g, "g", f32, (B, T, H, K), dev)
    _need(beta, "beta", f32, (B, T, H), dev)
    _need(Akk, "Akk", f32, (B, T, H, CHUNK), dev)
    _need(h, "h", bf, (B, NT, H, K, V), dev)
    _need(dh, "dh", bf, (B, NT, H, K, V), dev)
    out = dict(dq=torch.empty(B, T, H, K, device=dev, dtype=bf), dk=torch.empty(B, T, H, K, device=dev, dtype=bf),
               dv=torch.empty(B, T, H, V, device=dev, dtype=bf), dg=torch.empty_like(g),
               dbeta=torch.empty(B, T, H, device=dev, dtype=f32))
    P = _lib.ptr
    st = _lib.load().fdr_chunk_bwd_original(P(q), P(k), P(v), P(v_new), P(dO), P(dR), P(g), P(beta), P(Akk), P(h),
                                            P(dh), P(out["dq"]), P(out["dk"]), P(out["dv"]), P(out["dg"]),
                                            P(out["dbeta"]), B, T, H, K, V, CHUNK, float(scale),
                                            _lib.stream_handle(dev))
    _lib.check(st, "fdr_chunk_bwd_original")
    return out


def _chunk_bwd_gate_fold(q, k, v, v_new, dO, dR, g, gate_mode, Akk, h, dh, scale, beta, b, fold, beta_sigmoid=0.0,
                         hvf=0, H=None, mv=None):
    """chunk_bwd (KDA) with the gate backward folded into the dg stores; ``mv``: a packed
    batch whose sequences start anywhere (a mapped ``Varlen``)."""
    B, T, HQ, K = q.shape
    H = HQ if H is None else H
    V = V_SUPPORTED
    dev = q.device
    bf, f32 = torch.bfloat16, torch.float32
    if gate_mode != GATE_VECTOR or b is not None:
        raise ValueError("the folded gate backward is KDA's (vector gate, scalar beta)")
    g_raw, A_log, dt_bias, lb = fold["g_raw"], fold.get("A_log"), fold.get("dt_bias"), fold.get("lower_bound")
    raw = g_raw if g_raw.dtype in (bf, f32) else g_raw.float()
    raw = raw.contiguous()
    _need(raw, "g_raw", raw.dtype, (B, T, H, K), dev)
    if lb is None and A_log is None:
        raise ValueError("A_log is required when lower_bound is not set")
    a = None if A_log is None else _need(A_log.float().contiguous(), "A_log", f32, (H,), dev)
    dt = None if dt_bias is None else _need(dt_bias.float().contiguous(), "dt_bias", f32, (H * K,), dev)
    out = dict(dq=torch.empty(B, T, H, K, device=dev, dtype=bf),
               dk=torch.empty(B, T, H, K, device=dev, dtype=bf),
               dv=torch.empty(B, T, H, V, device=dev, dtype=bf),
               dg=torch.empty(B, T, H, K, device=dev, dtype=raw.dtype),
               dbeta=torch.empty(B, T, H, device=dev, dtype=f32), db=None, dw=None,
               dA_log=torch.empty(H, device=dev, dtype=f32) if A_log is not None else None,
               ddt_bias=torch.empty(H * K, device=dev, dtype=f32) if dt_bias is not None else None)
    lib = _lib.load()
    P = _lib.ptr
    args = (P(q), P(k), P(v), P(v_new), P(dO), P(dR), P(g), P(beta), P(Akk), P(h), P(dh), P(out["dq"]),
            P(out["dk"]), P(out["dv"]), P(out["dbeta"]), beta_sigmoid, P(raw), int(raw.dtype == bf), P(a), P(dt),
            int(lb is not None), 0.0 if lb is None else float(lb), P(out["dg"]), P(out["dA_log"]),
            P(out["ddt_bias"]))
    if mv is not None:
        ws = torch.empty(max(1, lib.fdr_chunk_bwd_gate_workspace_bytes(1, CHUNK * mv.NC, H) // 4), device=dev,
                         dtype=f32)
        st = lib.fdr_chunk_bwd_gate_fold_varlen(*args, P(ws), hvf, P(mv.cu_seqlens), P(mv.chunk_indices), mv.NC, H,
                                                HQ, K, V, CHUNK, float(scale), _lib.stream_handle(dev))
        _lib.check(st, "fdr_chunk_bwd_gate_fold_varlen")
        return out
    ws = torch.empty(max(1, lib.fdr_chunk_bwd_gate_workspace_bytes(B, T, H) // 4), device=dev, dtype=f32)
    st = lib.fdr_chunk_bwd_gate_fold(*args, P(ws), hvf, B, T, H, HQ, K, V, CHUNK, float(scale),
                                     _lib.stream_handle(dev))
    _lib.check(st, "fdr_chunk_bwd_gate_fold")
    return out


def prepare_wu(k, v, Akk, gate_mode, g=None, beta=None, b=None, w=None, q=None, want_qkg=False,
               want_aqk=False, scale=1.0, varlen=None, want_u=True):
    """WY factors (and qg/kg or Aqk) of every chunk.  Returns dict(w, u, qg, kg, Aqk).
    ``varlen``: a packed variable-length batch (``Varlen``).  ``want_u=False``: w (and, vector
    gates, optionally qg, kg) only, for ``fwd_h_u`` (u None; v and the write gate are not read)."""
    B, T, HQ, K = _rows(k, varlen)
    H, HQ = _group(v.shape[2] if v is not None and v.ndim == 4 else HQ, HQ)
    V = V_SUPPORTED
    dev = k.device
    bf, f32 = torch.bfloat16, torch.float32
    _need(k, "k", bf, (B, T, HQ, K), dev)
    _need(v, "v", bf, (B, T, H, V), dev)
    _need(Akk, "Akk", f32, (B, T, H, CHUNK), dev)
    if q is not None:
        _need(q, "q", bf, (B, T, HQ, K), dev)
    vec_b = b is not None
    if vec_b:
        _need(b, "b", bf, (B, T, H, K), dev)
        _need(w, "w", bf, (B, T, H, V), dev)
    else:
        _need(beta, "beta", f32, (B, T, H), dev)
    if gate_mode == GATE_VECTOR:
        _need(g, "g", f32, (B, T, H, K), dev)
    elif gate_mode == GATE_SCALAR:
        _need(g, "g", f32, (B, T, H), dev)
    elif gate_mode != GATE_NONE:
        raise ValueError("gate_mode must be 0, 1 or 2")
    if want_qkg and (q is None or gate_mode != GATE_VECTOR):
        raise ValueError("qg/kg need q and a vector gate")
    if want_aqk and (q is None or gate_mode == GATE_VECTOR):
        raise ValueError("Aqk is produced here for scalar / no-gate families only")
    if not want_u and varlen is not None:
        raise ValueError("want_u=False takes dense rows")
    out = dict(w=torch.empty(B, T, H, K, device=dev, dtype=bf),
               u=torch.empty(B, T, H, V, device=dev, dtype=bf) if want_u else None,
               qg=torch.empty(B, T, H, K, device=dev, dtype=bf) if want_qkg else None,
               kg=torch.empty(B, T, H, K, device=dev, dtype=bf) if want_qkg else None,
               Aqk=torch.empty(B, T, H, CHUNK, device=dev, dtype=f32) if want_aqk else None)
    P = _lib.ptr
    common = (P(q), P(k), P(v), P(g), int(gate_mode), P(beta), P(b), P(w), P(Akk), P(out["w"]), P(out["u"]),
              P(out["qg"]), P(out["kg"]), P(out["Aqk"]))
    mv = _mapped(varlen)
    if mv is not None:
        st = _lib.load().fdr_prepare_wu_varlen(*common, P(mv.cu_seqlens), P(mv.chunk_indices), mv.NC, H, HQ, K, V,
                                               CHUNK, float(scale), _lib.stream_handle(dev))
        _lib.check(st, "fdr_prepare_wu_varlen")
        return out
    st = _lib.load().fdr_prepare_wu(*common, B, T, H, HQ, K, V, CHUNK, float(scale), _lib.stream_handle(dev))
    _lib.check(st, "fdr_prepare_wu")
    return out


def fwd_h(k, w, u, g, gate_mode, h0=None, want_final=False, value_block=0, method="auto",
          chunk_offsets=None, state_v_first=False, varlen=None):
    """Forward state scan.  Returns (h [B,NT,H,K,V] bf16, v_new [B,T,H,V] bf16, final fp32|None).
    ``method``, ``chunk_offsets`` and ``varlen`` as for ``state_bwd`` (h0 / final per sequence)."""
    B, T, HQ, K = _rows(k, varlen)
    H, HQ = _group(w.shape[2] if w is not None and w.ndim == 4 else HQ, HQ)
    V = V_SUPPORTED
    dev = k.device
    bf, f32 = torch.bfloat16, torch.float32
    _need(k, "k", bf, (B, T, HQ, K), dev)
    _need(w, "w", bf, (B, T, H, K), dev)
    _need(u, "u", bf, (B, T, H, V), dev)
    if gate_mode == GATE_VECTOR:
        _need(g, "g", f32, (B, T, H, K), dev)
    elif gate_mode == GATE_SCALAR:
        _need(g, "g", f32, (B, T, H), dev)
    elif gate_mode != GATE_NONE:
        raise ValueError("gate_mode must be 0, 1 or 2")
    if varlen is not None:
        if chunk_offsets is not None:
            raise ValueError("pass chunk_offsets or varlen, not both")
        co, N, NT = varlen.chunk_offsets, varlen.N, varlen.NC
    else:
        co, N = _chunk_offsets(chunk_offsets, B, T, dev)
        NT = T // CHUNK
    if h0 is not None:
        _need(h0, "h0", f32, (N, H, K, V), dev)
    if value_block not in (0, 16, 32, 64):
        raise ValueError("value_block must be 0, 16, 32 or 64")
    vf = int(bool(state_v_first))
    h = torch.empty(B, NT, H, K, V, device=dev, dtype=bf)
    vnew = torch.empty(B, T, H, V, device=dev, dtype=bf)
    ht = torch.empty(N, H, K, V, device=dev, dtype=f32) if want_final else None
    P = _lib.ptr
    if co is not None:
        if method == "affine":
            raise ValueError("the affine-step form takes equal-length rows, not chunk_offsets")
        cu = _mapped(varlen)
        st = _lib.load().fdr_fwd_h_varlen(P(k), P(w), P(u), P(g), int(gate_mode), P(h0), P(h), P(vnew), P(ht),
                                          vf, P(co), None if cu is None else P(cu.cu_seqlens), N, NT, H, HQ, K, V,
                                          CHUNK, int(value_block), _lib.stream_handle(dev))
        _lib.check(st, "fdr_fwd_h_varlen")
        return h, vnew, ht
    if _use_affine(method, B, H, NT) and HQ == H:
        vb = value_block or AFFINE_VALUE_BLOCK
        step, offset = _affine_workspace(B, NT, H, dev)
        lib = _lib.load()
        st = lib.fdr_affine_prep_fwd(P(k), P(w), P(u), P(g), int(gate_mode), P(step), P(offset), B, T, H, K, V,
                                     CHUNK, _lib.stream_handle(dev))
        _lib.check(st, "fdr_affine_prep_fwd")
        arr, n = _lib.problems(_lib.ScanProblem, [_lib.ScanProblem(
            P(step), P(offset), P(g), P(h0), P(h), P(ht), int(gate_mode), 0, vf)])
        _lib.check(lib.fdr_affine_scan(arr, n, B, T, H, K, V, CHUNK, int(vb), _lib.stream_handle(dev)),
                   "fdr_affine_scan")
        arr, n = _lib.problems(_lib.SideProblem, [_lib.SideProblem(P(w), P(h), P(u), None, P(vnew), -1.0)])
        _lib.check(lib.fdr_affine_side(arr, n, B, T, H, K, V, CHUNK, _lib.stream_handle(dev)), "fdr_affine_side")
        return h, vnew, ht
    st = _lib.load().fdr_fwd_h(P(k), P(w), P(u), P(g), int(gate_mode), P(h0), P(h), P(vnew), P(ht), vf, B, T, H, HQ,
                               K, V, CHUNK, int(value_block), _lib.stream_handle(dev))
    _lib.check(st, "fdr_fwd_h")
    return h, vnew, ht


def group_sum(x, HQ):
    """dq / dk of grouped value heads summed over each q / k head's group (fdr_group_sum):
    x bf16 [B, T, HV, K] with HV = G HQ, value head j of group h at h G + j (FLA's head map);
    returns bf16 [B, T, HQ, K], each sum in fp32."""
    B, T, HV, K = x.shape
    if HV % HQ:
        raise ValueError(f"value heads ({HV}) must be a multiple of the q/k heads ({HQ})")
    _need(x, "x", torch.bfloat16, (B, T, HV, K), x.device)
    if K != K_SUPPORTED:
        raise ValueError(f"K must be {K_SUPPORTED}")
    out = torch.empty(B, T, HQ, K, device=x.device, dtype=torch.bfloat16)
    P = _lib.ptr
    _lib.check(_lib.load().fdr_group_sum(P(x), P(out), B * T, HQ, HV // HQ, K, _lib.stream_handle(x.device)),
               "fdr_group_sum")
    return out


def fwd_h_u(k, w, v, Akk, g, gate_mode, beta=None, w_gate=None, h0=None, want_final=False, value_block=0,
            state_v_first=False, b=None, kg=None):
    """``fwd_h`` with u formed in-kernel (fdr_fwd_h_u): u = Akk (beta v), or Akk (w_gate v) for
    GDN2, from the same MFMA sequence as ``prepare_wu``, so h, v_new and the final state are
    the bits of ``prepare_wu`` + ``fwd_h``.  k is the raw k (a vector gate's kg formed in-kernel
    with ``prepare_wu``'s rounding); w as ``prepare_wu(..., want_u=False)`` returns it, or None:
    then w = Akk (beta k 2^g), or Akk (b k 2^g) for GDN2 (``b``), is formed in-kernel too, as
    ``prepare_wu`` forms it.  ``kg`` (vector gate, w given): ``prepare_wu``'s kg, read instead
    of formed (k is then not read).  Returns (h, v_new, final|None)."""
    B, T, HQ, K = _dims(k)
    H, HQ = _group(v.shape[2] if v is not None and v.ndim == 4 else HQ, HQ)
    V = V_SUPPORTED
    dev = k.device
    bf, f32 = torch.bfloat16, torch.float32
    _need(k, "k", bf, (B, T, HQ, K), dev)
    if w is not None:
        _need(w, "w", bf, (B, T, H, K), dev)
    elif w_gate is not None:
        _need(b, "b", bf, (B, T, H, K), dev)
    if kg is not None:
        if gate_mode != GATE_VECTOR or w is None:
            raise ValueError("kg is read for a vector gate with w given")
        _need(kg, "kg", bf, (B, T, H, K), dev)
    _need(v, "v", bf, (B, T, H, V), dev)
    _need(Akk, "Akk", f32, (B, T, H, CHUNK), dev)
    if gate_mode == GATE_VECTOR:
        _need(g, "g", f32, (B, T, H, K), dev)
    elif gate_mode == GATE_SCALAR:
        _need(g, "g", f32, (B, T, H), dev)
    elif gate_mode != GATE_NONE:
        raise ValueError("gate_mode must be 0, 1 or 2")
    if w_gate is not None:
        if gate_mode != GATE_VECTOR:
            raise ValueError("w_gate (GDN2) takes the vector gate")
        _need(w_gate, "w_gate", bf, (B, T, H, V), dev)
    else:
        _need(beta, "beta", f32, (B, T, H), dev)
    if h0 is not None:
        _need(h0, "h0", f32, (B, H, K, V), dev)
    if value_block not in (0, 16, 32, 64):
        raise ValueError("value_block must be 0, 16, 32 or 64")
    NT = T // CHUNK
    h = torch.empty(B, NT, H, K, V, device=dev, dtype=bf)
    vnew = torch.empty(B, T, H, V, device=dev, dtype=bf)
    ht = torch.empty(B, H, K, V, device=dev, dtype=f32) if want_final else None
    P = _lib.ptr
    st = _lib.load().fdr_fwd_h_u(P(k), P(kg), P(w), P(v), P(g), int(gate_mode), P(beta), P(b if w is None else None),
                                 P(w_gate), P(Akk), P(h0), P(h), P(vnew), P(ht), int(bool(state_v_first)), B, T, H,
                                 HQ, K, V, CHUNK, int(value_block), _lib.stream_handle(dev))
    _lib.check(st, "fdr_fwd_h_u")
    return h, vnew, ht


def paired_recurrences(q, k, w, g, gate_mode, dO, scale, v, Akk, value_block, aqk=None, beta=None, b=None,
                       w_gate=None, qg=None, kg=None, raw_qk=False, h0=None, dht=None, want_dh0=True,
                       state_v_first=False):
    """``state_bwd`` (direct) and ``fwd_h_u`` in one launch (fdr_paired_recurrences): the
    state recurrence's work-groups and the scan's side by side, with the same bits as the two
    calls.  q / k are the raw ones (the scan's k).  Scalar / no gate: w as ``prepare_wu``
    writes it, Aqk formed by the state recurrence (``aqk`` None).  Vector gate: ``aqk``, and
    either ``qg`` / ``kg`` / ``w`` as ``prepare_wu`` wrote them (the state reads them, the scan
    reads kg), or ``raw_qk`` at 64-wide tiles (qg / kg formed in both; w given, or None to form
    it from ``beta`` or GDN2's ``b``).  GDN2 passes ``w_gate``, the others ``beta``.
    Returns ((dh, dR, dh0|None), (h, v_new, None))."""
    B, T, HQ, K = _dims(q)
    H, HQ = _group(v.shape[2] if v.ndim == 4 else HQ, HQ)
    V = V_SUPPORTED
    dev = q.device
    bf, f32 = torch.bfloat16, torch.float32
    for x, n in ((q, "q"), (k, "k")):
        _need(x, n, bf, (B, T, HQ, K), dev)
    _need(v, "v", bf, (B, T, H, V), dev)
    _need(dO, "dO", bf, (B, T, H, V), dev)
    _need(Akk, "Akk", f32, (B, T, H, CHUNK), dev)
    if gate_mode == GATE_VECTOR:
        _need(g, "g", f32, (B, T, H, K), dev)
        _need(aqk, "Aqk", f32, (B, T, H, CHUNK), dev)
    elif gate_mode in (GATE_SCALAR, GATE_NONE):
        if gate_mode == GATE_SCALAR:
            _need(g, "g", f32, (B, T, H), dev)
        if raw_qk or qg is not None or kg is not None:
            raise ValueError("scalar / no gate: the raw q / k")
        if aqk is not None:
            _need(aqk, "Aqk", f32, (B, T, H, CHUNK), dev)
    else:
        raise ValueError("gate_mode must be 0, 1 or 2")
    if w is not None:
        _need(w, "w", bf, (B, T, H, K), dev)
    elif not raw_qk or gate_mode != GATE_VECTOR:
        raise ValueError("w is formed in-kernel only with raw_qk")
    if w_gate is not None:
        if gate_mode != GATE_VECTOR:
            raise ValueError("w_gate (GDN2) takes the vector gate")
        _need(w_gate, "w_gate", bf, (B, T, H, V), dev)
        if w is None:
            _need(b, "b", bf, (B, T, H, K), dev)
    else:
        _need(beta, "beta", f32, (B, T, H), dev)
    if gate_mode == GATE_VECTOR and not raw_qk:
        _need(qg, "qg", bf, (B, T, H, K), dev)
        _need(kg, "kg", bf, (B, T, H, K), dev)
    if value_block not in (16, 32, 64) or (raw_qk and value_block != 64):
        raise ValueError("value_block must be 16, 32 or 64 (64 with raw_qk)")
    if h0 is not None:
        _need(h0, "h0", f32, (B, H, K, V), dev)
    if dht is not None:
        _need(dht, "dht", f32, (B, H, K, V), dev)
    NT = T // CHUNK
    dh = torch.empty(B, NT, H, K, V, device=dev, dtype=bf)
    dr = torch.empty(B, T, H, V, device=dev, dtype=bf)
    dh0 = torch.empty(B, H, K, V, device=dev, dtype=f32) if want_dh0 else None
    h = torch.empty(B, NT, H, K, V, device=dev, dtype=bf)
    vnew = torch.empty(B, T, H, V, device=dev, dtype=bf)
    P = _lib.ptr
    prepared = gate_mode == GATE_VECTOR and not raw_qk
    st = _lib.load().fdr_paired_recurrences(
        P(qg if prepared else q), P(kg if prepared else k), P(w), P(k), P(kg if prepared else None), P(g),
        int(gate_mode), P(beta), P(b if w is None else None), P(w_gate), P(v), P(Akk), P(aqk), P(dO), P(dht), P(h0),
        P(dh), P(dr), P(dh0), P(h), P(vnew), None, int(bool(raw_qk)), int(bool(state_v_first)), B, T, H, HQ, K, V,
        CHUNK, float(scale), int(value_block), _lib.stream_handle(dev))
    _lib.check(st, "fdr_paired_recurrences")
    return (dh, dr, dh0), (h, vnew, None)


def scalar_bwd(q, k, v, g, gate_mode, beta, Akk, dO, scale, value_block, aqk_in_prepare, dht=None, h0=None,
               want_dh0=True, beta_sigmoid=0.0, state_v_first=False):
    """GDN / DeltaNet recompute-policy backward in one library call (fdr_scalar_bwd):
    ``prepare_wu`` (w, and Aqk with ``aqk_in_prepare``), ``paired_recurrences`` at
    ``value_block`` and ``chunk_bwd``, with the same bits as those three calls and one
    allocation for the six intermediates (w, Aqk, dh, dR, h, v_new) instead of six.  Dense rows.
    Returns (dict(dq, dk, dv [per value head], dg | None, dbeta, db=None, dw=None), dh0 | None)."""
    B, T, HQ, K = _dims(q)
    H = v.shape[2]
    V = V_SUPPORTED
    dev = q.device
    bf, f32 = torch.bfloat16, torch.float32
    if gate_mode not in (GATE_SCALAR, GATE_NONE):
        raise ValueError("scalar_bwd: gate_mode 0 or 1")
    if H % HQ:
        raise ValueError("value heads must be a multiple of q / k heads")
    _need(q, "q", bf, (B, T, HQ, K), dev)
    _need(k, "k", bf, (B, T, HQ, K), dev)
    _need(v, "v", bf, (B, T, H, V), dev)
    _need(dO, "dO", bf, (B, T, H, V), dev)
    _need(beta, "beta", f32, (B, T, H), dev)
    _need(Akk, "Akk", f32, (B, T, H, CHUNK), dev)
    if gate_mode == GATE_SCALAR:
        _need(g, "g", f32, (B, T, H), dev)
    if dht is not None:
        _need(dht, "dht", f32, (B, H, K, V), dev)
    if h0 is not None:
        _need(h0, "h0", f32, (B, H, K, V), dev)
    lib = _lib.load()
    ws = torch.empty(lib.fdr_scalar_bwd_workspace_bytes(B, T, H, K, V, CHUNK), device=dev, dtype=torch.uint8)
    out = dict(dq=torch.empty(B, T, H, K, device=dev, dtype=bf), dk=torch.empty(B, T, H, K, device=dev, dtype=bf),
               dv=torch.empty(B, T, H, V, device=dev, dtype=bf),
               dg=torch.empty(B, T, H, device=dev, dtype=f32) if gate_mode == GATE_SCALAR else None,
               dbeta=torch.empty(B, T, H, device=dev, dtype=f32), db=None, dw=None)
    dh0 = torch.empty(B, H, K, V, device=dev, dtype=f32) if want_dh0 else None
    P = _lib.ptr
    st = lib.fdr_scalar_bwd(P(q), P(k), P(v), P(g), int(gate_mode), P(beta), P(Akk), P(dO), P(dht), P(h0),
                            P(out["dq"]), P(out["dk"]), P(out["dv"]), P(out["dg"]), P(out["dbeta"]), P(dh0), P(ws),
                            ws.numel(), float(beta_sigmoid or 0.0), int(bool(aqk_in_prepare)),
                            int(bool(state_v_first)), B, T, H, HQ, K, V, CHUNK, float(scale), int(value_block),
                            _lib.stream_handle(dev))
    _lib.check(st, "fdr_scalar_bwd")
    return out, dh0


def default_tile(N, H):
    """Value-tile width the recurrence kernels take by default for N rows of H heads (the C
    library's rule): the narrowest of 16 / 32 at which one launch holds at most 256 work-groups,
    64 beyond."""
    BH = N * H
    return 16 if BH * 8 <= 256 else 32 if BH * 4 <= 256 else 64


def fwd_h_wy_pays(N, H, gate_mode, varlen=None):
    """Whether ``fwd_h_wy`` beats ``prepare_wu`` + ``fwd_h`` for N rows (sequences) of H heads.
    Each value-tile work-group forms the whole w (and, for a vector gate, every qg / kg / E
    exponential) of its chunk, so that work is repeated once per value tile of a head (tile
    widths: ``default_tile``).  Measured: at 64-wide tiles the sweep wins for every family; at
    32-wide ones the scalar / no-gate families still win and the vector gates lose; at 16-wide
    ones all lose.
    A packed batch (``varlen``) scans for as long as its longest sequence, which then carries
    the sweep's extra work on every one of its chunks while the pair's ``prepare_wu`` spreads
    it over all chunks: it takes the sweep only when its sequences are near one length
    (longest x N <= 1.5 x all chunks; ten sequences of 300-8192 tokens measured 3.86 ms fused
    vs 3.64 ms with the pair)."""
    if varlen is not None and varlen.max_chunks * varlen.N > 1.5 * varlen.NC:
        return False
    if gate_mode == GATE_VECTOR:
        return default_tile(N, H) == 64
    return default_tile(N, H) >= 32


def fwd_h_wy(k, v, Akk, g, gate_mode, beta=None, q=None, b=None, w=None, h0=None, want_final=False,
             value_block=0, state_v_first=False, varlen=None):
    """``prepare_wu`` (w, u; qg, kg for a vector gate) and the direct ``fwd_h`` in one sweep.
    Operands as for ``prepare_wu`` (raw q / k; scalar beta, or GDN2's b and w_gate).  Returns
    dict(w, qg, kg, h, v_new, final) with the bits of that pair (qg / kg None unless
    gate_mode 2, final None unless want_final); u is not materialized.  ``varlen`` as for
    ``fwd_h`` (h0 / final per sequence)."""
    B, T, HQ, K = _rows(k, varlen)
    H, HQ = _group(v.shape[2] if v.ndim == 4 else HQ, HQ)
    V = V_SUPPORTED
    dev = k.device
    bf, f32 = torch.bfloat16, torch.float32
    vec = gate_mode == GATE_VECTOR
    _need(k, "k", bf, (B, T, HQ, K), dev)
    _need(v, "v", bf, (B, T, H, V), dev)
    _need(Akk, "Akk", f32, (B, T, H, CHUNK), dev)
    if b is not None:
        if not vec or HQ != H:
            raise ValueError("b / w_gate (GDN2) take the vector gate and one q/k head per value head")
        _need(b, "b", bf, (B, T, H, K), dev)
        _need(w, "w_gate", bf, (B, T, H, V), dev)
    else:
        _need(beta, "beta", f32, (B, T, H), dev)
    if vec:
        _need(g, "g", f32, (B, T, H, K), dev)
        _need(q, "q", bf, (B, T, HQ, K), dev)
    elif gate_mode == GATE_SCALAR:
        _need(g, "g", f32, (B, T, H), dev)
    elif gate_mode != GATE_NONE:
        raise ValueError("gate_mode must be 0, 1 or 2")
    if varlen is not None:
        co, N, NT = varlen.chunk_offsets, varlen.N, varlen.NC
    else:
        co, N, NT = None, B, T // CHUNK
    if h0 is not None:
        _need(h0, "h0", f32, (N, H, K, V), dev)
    if value_block not in (0, 16, 32, 64):
        raise ValueError("value_block must be 0, 16, 32 or 64")
    vf = int(bool(state_v_first))
    wo = torch.empty(B, T, H, K, device=dev, dtype=bf)
    qg = torch.empty(B, T, H, K, device=dev, dtype=bf) if vec else None
    kg = torch.empty(B, T, H, K, device=dev, dtype=bf) if vec else None
    h = torch.empty(B, NT, H, K, V, device=dev, dtype=bf)
    vnew = torch.empty(B, T, H, V, device=dev, dtype=bf)
    ht = torch.empty(N, H, K, V, device=dev, dtype=f32) if want_final else None
    P = _lib.ptr
    args = (P(q if vec else None), P(k), P(v), P(g), int(gate_mode), P(beta), P(b), P(w), P(Akk), P(h0), P(wo),
            P(qg), P(kg), P(h), P(vnew), P(ht), vf)
    if co is not None:
        cu = _mapped(varlen)
        st = _lib.load().fdr_fwd_h_wy_varlen(*args, P(co), None if cu is None else P(cu.cu_seqlens), N, NT, H, HQ,
                                             K, V, CHUNK, int(value_block), _lib.stream_handle(dev))
        _lib.check(st, "fdr_fwd_h_wy_varlen")
    else:
        st = _lib.load().fdr_fwd_h_wy(*args, B, T, H, HQ, K, V, CHUNK, int(value_block), _lib.stream_handle(dev))
        _lib.check(st, "fdr_fwd_h_wy")
    return dict(w=wo, qg=qg, kg=kg, h=h, v_new=vnew, final=ht)


def matrix_intra(q, k, g, dAqk, dAkk, dq, dk, db, dg, beta=None, b=None, beta_complete=False, varlen=None):
    """Matrix intra VJP added in place into fp32 (dq, dk, db, dg); returns them.  ``varlen``:
    a packed variable-length batch (``Varlen``)."""
    B, T, HQ, K = _rows(q, varlen)
    if varlen is None and T % CHUNK:
        raise ValueError("T must be a multiple of 64 (pass cu_seqlens for ragged rows)")
    H, HQ = _group(dq.shape[2] if dq is not None and dq.ndim == 4 else HQ, HQ)
    dev = q.device
    bf, f32 = torch.bfloat16, torch.float32
    _need(q, "q", bf, (B, T, HQ, K), dev)
    _need(k, "k", bf, (B, T, HQ, K), dev)
    _need(g, "g", f32, (B, T, H, K), dev)
    _need(dAqk, "dAqk", f32, (B, T, H, CHUNK), dev)
    _need(dAkk, "dAkk", f32, (B, T, H, CHUNK), dev)
    for x, n in ((dq, "dq"), (dk, "dk"), (dg, "dg")):
        _need(x, n, f32, (B, T, H, K), dev)
    if (beta is None) == (b is None):
        raise ValueError("exactly one of beta (scalar) / b (vector erase gate) is required")
    if b is not None:
        _need(b, "b", bf, (B, T, H, K), dev)
        _need(db, "db", f32, (B, T, H, K), dev)
    else:
        _need(beta, "beta", f32, (B, T, H), dev)
        _need(db, "db", f32, (B, T, H), dev)
    P = _lib.ptr
    mv = _mapped(varlen)
    if mv is not None:
        st = _lib.load().fdr_matrix_intra_varlen(P(q), P(k), P(g), P(beta), P(b), P(dAqk), P(dAkk), P(dq), P(dk),
                                                 P(db), P(dg), P(mv.cu_seqlens), P(mv.chunk_indices), mv.NC, H, HQ,
                                                 K, CHUNK, int(bool(beta_complete)), _lib.stream_handle(dev))
        _lib.check(st, "fdr_matrix_intra_varlen")
        return dq, dk, db, dg
    st = _lib.load().fdr_matrix_intra(P(q), P(k), P(g), P(beta), P(b), P(dAqk), P(dAkk), P(dq), P(dk), P(db),
                                      P(dg), B, T, H, HQ, K, CHUNK, int(bool(beta_complete)), _lib.stream_handle(dev))
    _lib.check(st, "fdr_matrix_intra")
    return dq, dk, db, dg


def fwd_prepare(q, k, g, gate_mode, beta=None, b=None, scale=1.0, varlen=None):
    """Forward intra matrices.  Returns (gc fp32 | None, Aqk fp32, Akk fp32).
    ``varlen``: a packed variable-length batch (``Varlen``)."""
    B, T, HQ, K = _rows(q, varlen)
    side = beta if beta is not None else b
    H, HQ = _group(side.shape[2] if side is not None and side.ndim >= 3 else HQ, HQ)
    dev = q.device
    bf, f32 = torch.bfloat16, torch.float32
    _need(q, "q", bf, (B, T, HQ, K), dev)
    _need(k, "k", bf, (B, T, HQ, K), dev)
    if gate_mode == GATE_VECTOR:
        _need(g, "g", f32, (B, T, H, K), dev)
    elif gate_mode == GATE_SCALAR:
        _need(g, "g", f32, (B, T, H), dev)
    elif gate_mode != GATE_NONE:
        raise ValueError("gate_mode must be 0, 1 or 2")
    if b is not None:
        if gate_mode != GATE_VECTOR:
            raise ValueError("a vector erase gate needs a vector decay gate")
        _need(b, "b", bf, (B, T, H, K), dev)
    else:
        _need(beta, "beta", f32, (B, T, H), dev)
    gc = torch.empty_like(g) if gate_mode != GATE_NONE else None
    Aqk = torch.empty(B, T, H, CHUNK, device=dev, dtype=f32)
    Akk = torch.empty(B, T, H, CHUNK, device=dev, dtype=f32)
    P = _lib.ptr
    common = (P(q), P(k), P(g), int(gate_mode), P(beta), P(b), P(gc), P(Aqk), P(Akk))
    mv = _mapped(varlen)
    if mv is not None:
        st = _lib.load().fdr_fwd_prepare_varlen(*common, P(mv.cu_seqlens), P(mv.chunk_indices), mv.NC, H, HQ, K,
                                                CHUNK, float(scale), _lib.stream_handle(dev))
        _lib.check(st, "fdr_fwd_prepare_varlen")
        return gc, Aqk, Akk
    st = _lib.load().fdr_fwd_prepare(*common, B, T, H, HQ, K, CHUNK, float(scale), _lib.stream_handle(dev))
    _lib.check(st, "fdr_fwd_prepare")
    return gc, Aqk, Akk


def fwd_o(q, gc, gate_mode, Aqk, h, v_new, scale, varlen=None):
    """Forward output o = scale (q 2^gc) h + Aqk v_new (bf16).  ``varlen``: a packed
    variable-length batch (``Varlen``; h has ``varlen.NC`` chunks)."""
    B, T, HQ, K = _rows(q, varlen)
    H, HQ = _group(Aqk.shape[2] if Aqk is not None and Aqk.ndim == 4 else HQ, HQ)
    V = V_SUPPORTED
    dev = q.device
    bf, f32 = torch.bfloat16, torch.float32
    _need(q, "q", bf, (B, T, HQ, K), dev)
    if gate_mode == GATE_VECTOR:
        _need(gc, "gc", f32, (B, T, H, K), dev)
    elif gate_mode == GATE_SCALAR:
        _need(gc, "gc", f32, (B, T, H), dev)
    elif gate_mode != GATE_NONE:
        raise ValueError("gate_mode must be 0, 1 or 2")
    _need(Aqk, "Aqk", f32, (B, T, H, CHUNK), dev)
    _need(h, "h", bf, (B, T // CHUNK if varlen is None else varlen.NC, H, K, V), dev)
    _need(v_new, "v_new", bf, (B, T, H, V), dev)
    o = torch.empty(B, T, H, V, device=dev, dtype=bf)
    P = _lib.ptr
    common = (P(q), P(gc), int(gate_mode), P(Aqk), P(h), P(v_new), P(o))
    mv = _mapped(varlen)
    if mv is not None:
        st = _lib.load().fdr_fwd_o_varlen(*common, P(mv.cu_seqlens), P(mv.chunk_indices), mv.NC, H, HQ, K, V, CHUNK,
                                          float(scale), _lib.stream_handle(dev))
        _lib.check(st, "fdr_fwd_o_varlen")
        return o
    st = _lib.load().fdr_fwd_o(*common, B, T, H, HQ, K, V, CHUNK, float(scale), _lib.stream_handle(dev))
    _lib.check(st, "fdr_fwd_o")
    return o
