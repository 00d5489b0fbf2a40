"""The C-ABI library: loads, exports every symbol include/rewy_amd.h declares,
and validates arguments on the host (no GPU needed for any of these calls)."""
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
    st = lib.fdr_state_bwd(None, None, None, None, 2, None, None, None, None, None, None, None,
                           1, 128, 1, 64, 128, 64, 1.0, 0, None)
    assert st == HIP_ERROR_INVALID_VALUE
    # T not a multiple of 64
    st = lib.fdr_chunk_bwd(*([None] * 7), 2, *([None] * 13), 1, 100, 1, 128, 128, 64, 1.0, None)
    assert st == HIP_ERROR_INVALID_VALUE
    # null pointers with a valid shape
    st = lib.fdr_chunk_bwd(*([None] * 7), 2, *([None] * 13), 1, 128, 1, 128, 128, 64, 1.0, None)
    assert st == HIP_ERROR_INVALID_VALUE
    # matrix intra: chunk 32, then null operands
    st = lib.fdr_matrix_intra(*([None] * 11), 1, 128, 1, 128, 32, 0, None)
    assert st == HIP_ERROR_INVALID_VALUE
    st = lib.fdr_matrix_intra(*([None] * 11), 1, 128, 1, 128, 64, 0, None)
    assert st == HIP_ERROR_INVALID_VALUE


def test_host_wrappers_validate_before_launch():
    import torch
    from rewy_amd import ops
    q = torch.zeros(1, 128, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        ops.state_bwd(q, q, q, None, 0, q, 1.0, dv=q)
    with pytest.raises(ValueError, match="multiple of 64"):
        ops.chunk_bwd(q[:, :100], q, q, q, q, q, None, 0, None, None, None, 1.0)
