"""ctypes binding of librewy_hip.so (the C-ABI declared in include/rewy_amd.h).

The library is loaded after torch so that it binds to the HIP runtime torch
already has in the process (same soname).  A missing library is an error:
there is no fallback path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("librewy_hip.so")

# every symbol the header declares, with its ctypes signature
_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
SIGNATURES = {
    "fdr_state_bwd": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P],
    "fdr_state_bwd_raw_qk": [_P] * 13 + [_I] * 8 + [_F, _I, _P],
    "fdr_state_bwd_segmented": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I,
                                _I, _P, _P],
    "fdr_chunk_bwd": [_P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _I, _I,
                      _I, _I, _I, _I, _I, _I, _F, _P],
    "fdr_chunk_bwd_original": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P],
    "fdr_prepare_wu": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P],
    "fdr_fwd_h": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P],
    "fdr_fwd_h_u": [_P] * 5 + [_I] + [_P] * 8 + [_I] * 9 + [_P],
    "fdr_paired_recurrences": [_P] * 6 + [_I] + [_P] * 15 + [_I] * 9 + [_F, _I, _P],
    "fdr_scalar_bwd": [_P] * 4 + [_I] + [_P] * 12 + [ctypes.c_size_t, _F] + [_I] * 9 + [_F, _I, _P],
    "fdr_state_bwd_varlen": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F,
                             _I, _P],
    "fdr_fwd_h_varlen": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P],
    "fdr_fwd_h_wy": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I,
                     _I, _P],
    "fdr_fwd_h_wy_varlen": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I,
                            _I, _I, _I, _I, _I, _P],
    "fdr_fwd_prepare_varlen": [_P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P],
    "fdr_prepare_wu_varlen": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                              _F, _P],
    "fdr_fwd_o_varlen": [_P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P],
    "fdr_chunk_bwd_varlen": [_P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P,
                             _I, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P],
    "fdr_stream_probe": [_I, _P, _P, ctypes.c_longlong, _I, _P],
    "fdr_chunk_bwd_wy": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                         _I, _I, _F, _P],
    "fdr_matrix_intra": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P],
    "fdr_matrix_intra_varlen": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    "fdr_chunk_bwd_wy_varlen": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I,
                                _I, _I, _I, _I, _I, _F, _P],
    "fdr_gdn2_chunk_bwd_wy": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I,
                              _I, _I, _I, _I, _I, _F, _P],
    "fdr_gdn2_chunk_bwd_wy_varlen": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I,
                                     _P, _P, _I, _I, _I, _I, _I, _F, _P],
    "fdr_fwd_prepare": [_P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P],
    "fdr_fwd_o": [_P, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P],
    "fdr_affine_prep_bwd": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P],
    "fdr_affine_prep_fwd": [_P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    "fdr_affine_prep_pair": [_P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P],
    "fdr_kda_gate_fwd": [_P, _I, _P, _P, _I, _F, _P, _I, _I, _I, _I, _P],
    "fdr_kda_gate_bwd": [_P, _P, _I, _P, _P, _I, _F, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "fdr_beta_sigmoid_fwd": [_P, _I, _F, _P, ctypes.c_longlong, _P],
    "fdr_group_sum": [_P, _P, ctypes.c_longlong, _I, _I, _I, _P],
    "fdr_l2norm_fwd": [_P, _I, _P, _P, ctypes.c_longlong, _I, _F, _P],
    "fdr_l2norm_bwd": [_P, _I, _P, _P, _P, ctypes.c_longlong, _I, _P],
    "fdr_chunk_bwd_gate_fold": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _I, _P, _P, _I,
                                _F, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _P],
    "fdr_chunk_bwd_gate_fold_varlen": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _I, _P,
                                       _P, _I, _F, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P],
    "fdr_chunk_bwd_gate_fold_noalloc": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _I, _P,
                                        _P, _I, _F, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _P],
    "fdr_affine_scan": [_P, _I, _I, _I, _I, _I, _I, _I, _I, _P],
    "fdr_affine_side": [_P, _I, _I, _I, _I, _I, _I, _I, _P],
}


class ScanProblem(ctypes.Structure):
    """fdr_scan_problem (include/rewy_amd.h)."""
    _fields_ = [("step", _P), ("offset", _P), ("g", _P), ("initial", _P), ("states", _P),
                ("final_state", _P), ("gate_mode", _I), ("reverse", _I), ("state_v_first", _I)]


class SideProblem(ctypes.Structure):
    """fdr_side_problem (include/rewy_amd.h)."""
    _fields_ = [("x", _P), ("states", _P), ("addend", _P), ("row_gate", _P), ("out", _P), ("sign", _F)]


def problems(struct, items):
    """ctypes array of one or two problem structs (passed by pointer)."""
    arr = (struct * len(items))(*items)
    return arr, len(items)


_lib = None


class HipError(RuntimeError):
    pass


def load():
    """Load (once) and return the library handle."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401  -- bind to torch's HIP runtime first
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m rewy_amd.build` "
                               "(the HIP backward has no fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        lib.fdr_kda_gate_workspace_bytes.argtypes = [_I, _I, _I, _I]
        lib.fdr_kda_gate_workspace_bytes.restype = ctypes.c_size_t
        lib.fdr_state_bwd_segmented_workspace_bytes.argtypes = [_I, _I, _I]
        lib.fdr_state_bwd_segmented_workspace_bytes.restype = ctypes.c_size_t
        lib.fdr_chunk_bwd_gate_workspace_bytes.argtypes = [_I, _I, _I]
        lib.fdr_chunk_bwd_gate_workspace_bytes.restype = ctypes.c_size_t
        lib.fdr_scalar_bwd_workspace_bytes.argtypes = [_I] * 6
        lib.fdr_scalar_bwd_workspace_bytes.restype = ctypes.c_size_t
        _lib = lib
    return _lib


def check(status: int, what: str):
    if status != 0:
        raise HipError(f"{what} failed with hipError_t {status}")


def ptr(t):
    """Device pointer of a tensor as an int (or None: a null pointer); the c_void_p argtypes
    convert it at the call."""
    return None if t is None else t.data_ptr()


def stream_handle(device):
    """The current HIP stream of ``device`` (torch's, so the kernels order with torch's own
    work), as a raw handle.  The raw lookup costs ~0.3 us against ~5 us for
    torch.cuda.current_stream(device), which tiny backwards pay four times per call."""
    import torch
    idx = device.index if device.index is not None else torch.cuda.current_device()
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)     # torch's own fast path
    if raw is None:
        return torch.cuda.current_stream(idx).cuda_stream
    return raw(idx)
