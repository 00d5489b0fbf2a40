"""The C-ABI library: loads, exports every symbol include/rewy_amd.h declares,
and validates arguments on the host (no GPU needed for any of these calls)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIP_ERROR_INVALID_VALUE = 1


def _declared():
    text = (ROOT / "include" / "rewy_amd.h").read_text()
    return re.findall(r"hipError_t\s+(fdr_\w+)\s*\(", text)


def test_header_and_ctypes_table_agree():
    from rewy_amd import _lib
    assert sorted(_declared()) == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    from rewy_amd import _lib
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name


def test_entry_points_reject_unsupported_shapes_without_touching_the_gpu():
    from rewy_amd import _lib
    lib = _lib.load()
    # K = 64 (only 128 supported)
    st = lib.fdr_state_bwd(None, None, None, None, 2, None, None, None, None, None, None, None, 0,
                           1, 128, 1, 0, 64, 128, 64, 1.0, 0, None)
    assert st == HIP_ERROR_INVALID_VALUE
    # T not a multiple of 64
    st = lib.fdr_chunk_bwd(*([None] * 7), 2, *([None] * 11), 0.0, None, None, 0, 1, 100, 1, 0, 128, 128, 64, 1.0, None)
    assert st == HIP_ERROR_INVALID_VALUE
    # null pointers with a valid shape
    st = lib.fdr_chunk_bwd(*([None] * 7), 2, *([None] * 11), 0.0, None, None, 0, 1, 128, 1, 0, 128, 128, 64, 1.0, None)
    assert st == HIP_ERROR_INVALID_VALUE
    # matrix intra: chunk 32, then null operands
    st = lib.fdr_matrix_intra(*([None] * 11), 1, 128, 1, 0, 128, 32, 0, None)
    assert st == HIP_ERROR_INVALID_VALUE
    st = lib.fdr_matrix_intra(*([None] * 11), 1, 128, 1, 0, 128, 64, 0, None)
    assert st == HIP_ERROR_INVALID_VALUE


def test_new_entry_points_reject_bad_arguments_without_touching_the_gpu():
    from rewy_amd import _lib
    lib = _lib.load()
    # affine-step recurrences: K = 64; null operands; too many problems
    st = lib.fdr_affine_prep_bwd(*([None] * 4), 0, *([None] * 6), 1, 128, 1, 64, 128, 64, 1.0, None)
    assert st == HIP_ERROR_INVALID_VALUE
    st = lib.fdr_affine_prep_fwd(*([None] * 4), 0, None, None, 1, 128, 1, 128, 128, 64, None)
    assert st == HIP_ERROR_INVALID_VALUE
    probs = (_lib.ScanProblem * 3)()
    assert lib.fdr_affine_scan(probs, 3, 1, 128, 1, 128, 128, 64, 16, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fdr_affine_scan(probs, 1, 1, 128, 1, 128, 128, 64, 16, None) == HIP_ERROR_INVALID_VALUE  # null step
    sides = (_lib.SideProblem * 1)()
    assert lib.fdr_affine_side(sides, 1, 1, 100, 1, 128, 128, 64, None) == HIP_ERROR_INVALID_VALUE  # T % 64
    # gate kernels: K = 64, then no A_log without a lower bound
    st = lib.fdr_kda_gate_fwd(None, 0, None, None, 0, 0.0, None, 1, 64, 1, 64, None)
    assert st == HIP_ERROR_INVALID_VALUE
    assert lib.fdr_kda_gate_workspace_bytes(1, 64, 1, 64) == 0
    # l2norm: no rows
    assert lib.fdr_l2norm_fwd(None, 1, None, None, 0, 128, 1e-6, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fdr_l2norm_bwd(None, 1, None, None, None, 0, 128, None) == HIP_ERROR_INVALID_VALUE


def test_host_wrappers_validate_before_launch():
    import torch
    from rewy_amd import ops
    q = torch.zeros(1, 128, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        ops.state_bwd(q, q, q, None, 0, q, 1.0, dv=q)
    with pytest.raises(ValueError, match="multiple of 64"):
        ops.chunk_bwd(q[:, :100], q, q, q, q, q, None, 0, None, None, None, 1.0)


def test_backward_varlen_seam_validation():
    """cu_seqlens at the backward seam: the packed batch's chunk map (FLA's
    prepare_chunk_indices / prepare_chunk_offsets: each sequence cut into ceil(len / 64)
    chunks, an empty one owning none), sequences starting anywhere; malformed offsets are
    refused before any kernel runs."""
    import pytest
    import torch
    from rewy_amd.backends.backward import _varlen
    q = torch.zeros(1, 256, 1, 128)
    assert _varlen(q, {}) is None
    vl = _varlen(q, dict(cu_seqlens=torch.tensor([0, 64, 256])))
    assert vl.aligned and vl.chunk_offsets.tolist() == [0, 1, 4] and vl.NC == 4
    vl = _varlen(q, dict(cu_seqlens=torch.tensor([0, 100, 256])))
    assert not vl.aligned and (vl.N, vl.NC, vl.T) == (2, 5, 256)
    assert vl.chunk_offsets.tolist() == [0, 2, 5]
    assert vl.chunk_indices.tolist() == [[0, 0], [0, 1], [1, 0], [1, 1], [1, 2]]
    vl = _varlen(q, dict(cu_seqlens=torch.tensor([0, 64, 64, 65, 256])))
    assert vl.chunk_offsets.tolist() == [0, 1, 1, 2, 5]
    assert vl.chunk_indices.tolist() == [[0, 0], [2, 0], [3, 0], [3, 1], [3, 2]]
    with pytest.raises(ValueError, match="decrease"):
        _varlen(q, dict(cu_seqlens=torch.tensor([0, 128, 64, 256])))
    with pytest.raises(ValueError, match="rise"):
        _varlen(q, dict(cu_seqlens=torch.tensor([0, 64])))
    with pytest.raises(NotImplementedError):
        _varlen(q, dict(chunk_offsets=torch.tensor([0, 4])))


def _header_params():
    """Parameter kinds of every declared entry point, read from the header text."""
    text = (ROOT / "include" / "rewy_amd.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for name, params in re.findall(r"hipError_t\s+(fdr_\w+)\s*\(([^)]*)\)", text):
        kinds = []
        for prm in params.split(","):
            prm = " ".join(prm.split())
            if "*" in prm or prm.startswith("hipStream_t"):
                kinds.append("P")
            elif prm.startswith("float"):
                kinds.append("F")
            elif prm.startswith("long long"):
                kinds.append("L")
            elif prm.startswith("size_t"):
                kinds.append("Z")
            elif prm.startswith("int"):
                kinds.append("I")
            else:
                raise AssertionError(f"{name}: unknown parameter type {prm!r}")
        out[name] = kinds
    return out


def test_ctypes_signatures_match_the_header_parameter_by_parameter():
    import ctypes
    from rewy_amd import _lib
    kind = {ctypes.c_void_p: "P", ctypes.c_int: "I", ctypes.c_float: "F", ctypes.c_longlong: "L", ctypes.c_size_t: "Z"}
    for name, params in _header_params().items():
        got = [kind[t] for t in _lib.SIGNATURES[name]]
        assert got == params, (name, "".join(got), "".join(params))


def test_fused_scan_rule():
    """ops.fwd_h_wy_pays: by value-tile width (64-wide from 2 N H >= 256 work-groups, 32-wide
    from 4 N H >= 256) and, for a packed batch, by how far its longest sequence sets the scan"""
    import torch
    from rewy_amd import ops
    V, S, N0 = ops.GATE_VECTOR, ops.GATE_SCALAR, ops.GATE_NONE
    assert ops.fwd_h_wy_pays(8, 16, V) and ops.fwd_h_wy_pays(8, 16, S)
    assert not ops.fwd_h_wy_pays(2, 32, V) and ops.fwd_h_wy_pays(2, 32, S)      # 32-wide tiles
    assert not ops.fwd_h_wy_pays(2, 16, S) and not ops.fwd_h_wy_pays(2, 16, N0)  # 16-wide tiles
    even = ops.Varlen([0, 4096, 8192, 12288, 16384, 20480, 24576, 28672, 32768], "cpu")
    skewed = ops.Varlen(torch.tensor([0, 8192, 4096, 2048, 2048, 1024, 512, 300, 7000, 3000, 4548]).cumsum(0),
                        "cpu")
    assert even.max_chunks == 64 and skewed.max_chunks == 128 and skewed.NC == 514
    assert ops.fwd_h_wy_pays(even.N, 16, V, even)
    assert not ops.fwd_h_wy_pays(skewed.N, 16, V, skewed)


def test_side_by_side_rule():
    """ops.side_by_side_pays (recompute policy: the forward scan beside the segmented state
    recurrence) against the measured crossovers, and affine_pays stepping aside for it."""
    import torch
    from rewy_amd import ops
    sbs = ops.side_by_side_pays
    assert sbs(1, 16, 128) and sbs(1, 8, 128) and sbs(1, 16, 64)       # grid case 5 and its kin
    assert not sbs(1, 4, 128) and not sbs(1, 16, 32) and not sbs(1, 8, 64)   # the affine pair wins
    assert not sbs(2, 16, 128) and sbs(2, 16, 256)     # direct kernels until the segmented threshold
    assert not sbs(8, 16, 512)                         # the direct kernels fill the GPU
    meta = lambda B, T, H: torch.empty(B, T, H, 1, device="meta")
    assert not ops.affine_pays(meta(1, 8192, 16)) and ops.affine_pays(meta(1, 8192, 4))
    assert ops.affine_pays(meta(1, 2048, 16))


def test_paired_rule():
    """ops.paired_tile (recompute policy, vector gates: the direct state recurrence beside the
    direct forward scan): the narrowest of 32 / 64 at which each launch holds <= 128
    work-groups (17 <= B*H <= 32), 64-wide ones to B*H = 127, narrow rows at B*H <= 16."""
    from rewy_amd import ops
    V, S = ops.GATE_VECTOR, ops.GATE_SCALAR
    assert ops.paired_tile(2, 32, 128, V) == 64          # GDN2 configs[3]
    assert ops.paired_tile(2, 16, 64, V) == 32 and ops.paired_tile(1, 24, 256, V) == 32
    assert ops.paired_tile(1, 48, 128, V) == 64
    assert ops.paired_tile(1, 16, 512, V) == 0           # few heads, long rows: the side-by-side form
    assert ops.paired_tile(8, 16, 64, V) == 0            # B*H = 128: one after the other
    assert ops.paired_tile(1, 96, 64, V) == 64 and ops.paired_tile(1, 127, 64, S) == 64   # launches < 256 groups
    assert ops.paired_tile(1, 128, 64, V) == 0           # each recurrence fills the GPU
    assert ops.paired_tile(2, 32, 128, S) == 64 and ops.paired_tile(4, 16, 32, S) == 64   # before the fused sweep
    assert ops.paired_tile(2, 16, 32, S) == 32 and ops.paired_tile(1, 48, 64, ops.GATE_NONE) == 64
    assert ops.paired_tile(8, 16, 64, S) == 0
    # B*H <= 16: 16-wide tiles on rows of <= 8 chunks, of <= 128 from B*H = 12
    assert ops.paired_tile(1, 16, 32, V) == 16 and ops.paired_tile(2, 8, 64, S) == 16
    assert ops.paired_tile(1, 16, 8, ops.GATE_NONE) == 16 and ops.paired_tile(1, 2, 4, ops.GATE_NONE) == 16
    assert ops.paired_tile(1, 16, 129, S) == 0 and ops.paired_tile(1, 15, 32, V) == 16
    assert ops.paired_tile(1, 16, 128, V) == 16 and ops.paired_tile(1, 12, 128, V) == 16
    assert ops.paired_tile(1, 12, 129, V) == 0 and ops.paired_tile(1, 8, 16, V) == 0
    assert ops.paired_tile(1, 4, 32, V) == 0 and ops.paired_tile(1, 1, 8, S) == 16
    # 17 <= B*H < 24: 32-wide tiles
    assert ops.paired_tile(1, 20, 32, V) == 32 and ops.paired_tile(1, 17, 1024, S) == 32


def test_kernel_seams_validate_before_launch():
    """The kernel-level seams (state, WY, intra) reject what they do not take before any
    GPU work: chunk_indices without cu_seqlens, chunk_indices that do not match cu_seqlens,
    both gate kinds at once, other chunk sizes."""
    import pytest
    import torch
    from rewy_amd.backends.intra import chunk_gdn2_bwd_intra
    from rewy_amd.backends.state import chunk_gated_delta_rule_bwd_dhu
    from rewy_amd.backends.wy import chunk_gdn2_bwd_wy_dqkg_fused, chunk_kda_bwd_wy_dqkg_fused
    x = torch.zeros(1, 100, 2, 128)
    ci = torch.zeros(2, 2, dtype=torch.int32)
    cu = torch.tensor([0, 30, 100], dtype=torch.int32)
    with pytest.raises(NotImplementedError):
        chunk_kda_bwd_wy_dqkg_fused(x, x, x, x, x, x[..., 0], x, x, x, x, x, chunk_indices=ci)
    with pytest.raises(ValueError, match="chunk_indices must be"):
        chunk_gdn2_bwd_wy_dqkg_fused(x, x, x, x, x, x, x, x, x, x, x, x, cu_seqlens=cu,
                                     chunk_indices=torch.zeros(4, 2, dtype=torch.int32))
    with pytest.raises(NotImplementedError):
        chunk_gdn2_bwd_intra(x, x, x, x, x, x, x, x, x, x, chunk_size=32)
    with pytest.raises(ValueError, match="at most one"):
        chunk_gated_delta_rule_bwd_dhu(x, x, x, x, x, g=x[..., 0], gk=x)
    with pytest.raises(ValueError, match="batch size"):
        chunk_gated_delta_rule_bwd_dhu(torch.zeros(2, 100, 2, 128), x, x, x, x, cu_seqlens=cu)
    with pytest.raises(ValueError, match="GPU"):       # shapes pass; no device to run on
        chunk_gated_delta_rule_bwd_dhu(x, x, x, x, x, gk=x, cu_seqlens=cu)


def test_seam_and_pairing_entry_points_reject_bad_arguments_without_touching_the_gpu():
    """The kernel-level seams' packed-batch forms, GDN2's WY seam, the scan that forms u
    itself and the GVA group sum validate their shapes and pointers before any launch."""
    from rewy_amd import _lib
    lib = _lib.load()
    # K = 64 everywhere (only 128 supported), or no chunks / no row map
    assert lib.fdr_fwd_h_u(*([None] * 5), 2, *([None] * 8), 0, 1, 128, 1, 1, 64, 128, 64, 0,
                           None) == HIP_ERROR_INVALID_VALUE
    assert lib.fdr_fwd_h_u(*([None] * 5), 2, *([None] * 8), 0, 1, 128, 1, 1, 128, 128, 64, 0,
                           None) == HIP_ERROR_INVALID_VALUE            # null operands
    assert lib.fdr_state_bwd_raw_qk(*([None] * 13), 0, 1, 128, 1, 1, 64, 128, 64, 1.0, 0,
                                    None) == HIP_ERROR_INVALID_VALUE   # K = 64
    assert lib.fdr_state_bwd_raw_qk(*([None] * 13), 0, 1, 128, 1, 1, 128, 128, 64, 1.0, 0,
                                    None) == HIP_ERROR_INVALID_VALUE   # null operands
    assert lib.fdr_state_bwd_raw_qk(*([None] * 13), 0, 1, 100, 1, 1, 128, 128, 64, 1.0, 0,
                                    None) == HIP_ERROR_INVALID_VALUE   # T not whole chunks
    fake = ctypes.c_void_p(256)          # never dereferenced: each call is rejected before any launch
    # fdr_fwd_h_u: kg is read only for a vector gate with w given
    assert lib.fdr_fwd_h_u(fake, fake, fake, fake, fake, 1, fake, None, None, fake, None, fake, fake, None, 0, 1, 128,
                           1, 1, 128, 128, 64, 0, None) == HIP_ERROR_INVALID_VALUE     # scalar gate
    assert lib.fdr_fwd_h_u(fake, fake, None, fake, fake, 2, fake, None, None, fake, None, fake, fake, None, 0, 1, 128,
                           1, 1, 128, 128, 64, 0, None) == HIP_ERROR_INVALID_VALUE     # w NULL
    # fdr_state_bwd_raw_qk with w formed: exactly one of beta / b_gate, and Akk
    assert lib.fdr_state_bwd_raw_qk(fake, fake, None, fake, fake, fake, fake, fake, fake, None, fake, fake, None, 0,
                                    1, 128, 1, 1, 128, 128, 64, 1.0, 0, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fdr_state_bwd_raw_qk(fake, fake, None, fake, None, None, fake, fake, fake, None, fake, fake, None, 0,
                                    1, 128, 1, 1, 128, 128, 64, 1.0, 0, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fdr_state_bwd_raw_qk(fake, fake, None, fake, fake, None, None, fake, fake, None, fake, fake, None, 0,
                                    1, 128, 1, 1, 128, 128, 64, 1.0, 0, None) == HIP_ERROR_INVALID_VALUE
    # fdr_paired_recurrences (q, k, w, k_scan, kg, g, gate, beta, b_gate, w_gate, v, Akk, aqk, dO, dht,
    # h0, dh, dr, dh0, h, v_new, ht, raw_qk, vf, B, T, H, qk_heads, K, V, chunk, scale, value_block, stream)
    def paired(w=fake, kg=fake, gate=2, beta=fake, b_gate=None, w_gate=None, aqk=fake, raw=0, vb=32, T=128):
        return lib.fdr_paired_recurrences(fake, fake, w, fake, kg, fake, gate, beta, b_gate, w_gate, fake, fake, aqk,
                                          fake, None, None, fake, fake, None, fake, fake, None, raw, 0, 1, T, 2, 2,
                                          128, 128, 64, 1.0, vb, None)
    assert paired(vb=48) == HIP_ERROR_INVALID_VALUE                     # tile width
    assert paired(T=100) == HIP_ERROR_INVALID_VALUE                     # T not whole chunks
    assert paired(kg=None) == HIP_ERROR_INVALID_VALUE                   # vector gate, prepared: kg required
    assert paired(aqk=None) == HIP_ERROR_INVALID_VALUE                  # vector gate: Aqk required
    assert paired(raw=1) == HIP_ERROR_INVALID_VALUE                     # raw q / k: not with kg ...
    assert paired(raw=1, kg=None, vb=32) == HIP_ERROR_INVALID_VALUE     # ... and only at 64-wide tiles
    assert paired(raw=1, kg=None, w=None, beta=None, b_gate=None, w_gate=fake,
                  vb=64) == HIP_ERROR_INVALID_VALUE                     # GDN2 with w formed: b_gate required
    assert paired(gate=1, kg=None, w=None) == HIP_ERROR_INVALID_VALUE   # scalar gate: w required
    assert paired(gate=1, kg=None, raw=1) == HIP_ERROR_INVALID_VALUE    # scalar gate: no raw_qk
    assert paired(gate=1, w_gate=fake) == HIP_ERROR_INVALID_VALUE       # w_gate only with the vector gate
    # fdr_scalar_bwd (q, k, v, g, gate, beta, Akk, dO, dht, h0, dq, dk, dv, dg, dbeta, dh0, workspace,
    # workspace_bytes, beta_sigmoid, aqk_in_prepare, vf, B, T, H, qk_heads, K, V, chunk, scale, value_block, stream)
    need = lib.fdr_scalar_bwd_workspace_bytes(1, 128, 2, 128, 128, 64)
    assert need == 65536 + 65536 + 131072 + 65536 + 131072 + 65536     # w, Aqk, dh, dR, h, v_new
    assert lib.fdr_scalar_bwd_workspace_bytes(1, 100, 2, 128, 128, 64) == 0

    def scalar(gate=1, g=fake, dg=fake, ws=fake, nbytes=need, sig=0.0, vb=32, T=128, HQ=2):
        return lib.fdr_scalar_bwd(fake, fake, fake, g, gate, fake, fake, fake, None, None, fake, fake, fake, dg, fake,
                                  None, ws, nbytes, sig, 1, 0, 1, T, 2, HQ, 128, 128, 64, 1.0, vb, None)
    assert scalar(gate=2) == HIP_ERROR_INVALID_VALUE                     # GDN / DeltaNet only
    assert scalar(g=None) == HIP_ERROR_INVALID_VALUE                     # GDN: g required ...
    assert scalar(gate=0) == HIP_ERROR_INVALID_VALUE                     # ... DeltaNet: none
    assert scalar(dg=None) == HIP_ERROR_INVALID_VALUE                    # GDN: dg required
    assert scalar(vb=48) == HIP_ERROR_INVALID_VALUE                      # tile width
    assert scalar(T=100) == HIP_ERROR_INVALID_VALUE                      # T not whole chunks
    assert scalar(HQ=3) == HIP_ERROR_INVALID_VALUE                       # q / k heads do not divide H
    assert scalar(sig=-1.0) == HIP_ERROR_INVALID_VALUE                   # beta_sigmoid >= 0
    assert scalar(nbytes=need - 1) == HIP_ERROR_INVALID_VALUE            # workspace too small
    assert scalar(ws=ctypes.c_void_p(320)) == HIP_ERROR_INVALID_VALUE    # workspace not 256-byte aligned
    assert scalar(ws=None) == HIP_ERROR_INVALID_VALUE
    assert lib.fdr_group_sum(None, None, 16, 2, 2, 64, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fdr_group_sum(None, None, 0, 2, 2, 128, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fdr_gdn2_chunk_bwd_wy(*([None] * 19), 0, 1, 128, 1, 64, 128, 64, 1.0, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fdr_gdn2_chunk_bwd_wy_varlen(*([None] * 19), 0, None, None, 2, 1, 128, 128, 64, 1.0,
                                            None) == HIP_ERROR_INVALID_VALUE   # no row map
    assert lib.fdr_chunk_bwd_wy_varlen(*([None] * 17), 0, None, None, 2, 1, 1, 128, 128, 64, 1.0,
                                       None) == HIP_ERROR_INVALID_VALUE
    assert lib.fdr_matrix_intra_varlen(*([None] * 13), 0, 1, 1, 128, 64, 0, None) == HIP_ERROR_INVALID_VALUE


def test_integration_guide_ctypes_lines_match_the_bindings():
    """Every `lib.<entry>.argtypes = ...` line INTEGRATION.md shows a maintainer is the
    signature this package binds (rewy_amd/_lib.py), which test_header_and_ctypes_table_agree ties
    to include/rewy_amd.h."""
    import ctypes
    from rewy_amd import _lib
    env = {"P": ctypes.c_void_p, "I": ctypes.c_int, "F": ctypes.c_float, "ctypes": ctypes}
    pat = re.compile(r"lib\.(fdr_\w+)\.argtypes = (\[[^`]*?\](?:\s*[\*\+]\s*(?:\d+|\[[^`\]]*\]))*)")
    seen = 0
    for line in (ROOT / "INTEGRATION.md").read_text().splitlines():
        for name, expr in pat.findall(line):
            assert name in _lib.SIGNATURES, name
            assert list(eval(expr, env)) == list(_lib.SIGNATURES[name]), name
            seen += 1
    assert seen >= 10
