"""Explicit backend selection, the release envelope and the dispatch report.

Mirrors reference ``src/fast_delta_rule/runtime.py``: the same ``OPERATORS``
table (:14-19), ``Selection`` ContextVar (:21-27), counters ``record`` /
``stats`` (:31-37), ``configure`` / ``use_backend`` (:39-50), envelope
``rejection_reason`` (:75-106), router ``operator`` (:114-143) and
``assert_used`` (:145-149).  Importing this module imports no torch.

Differences, all forced by the platform:
* ``original`` routes to this package's PyTorch implementation of the original
  7-product formulation (``rewy_amd.original``) instead of FLA, which is not
  part of this build;
* ``check_baseline`` fingerprints this package's own HIP library against the
  sources it was built from (the reference fingerprints FLA's sources, :52-67).

One deliberate widening: packed variable-length batches (``cu_seqlens``) are
accepted by the optimized backend, which runs them as zero-padded batch rows
(``_compat.api._apply``); the reference's envelope rejects them.
"""
from collections import Counter
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass
from functools import lru_cache, wraps
import hashlib
import importlib
import inspect
import json
from pathlib import Path
import warnings

OPERATORS = {
    'kda': ('kda', 'chunk_kda'),
    'gdn': ('gdn', 'chunk_gated_delta_rule'),
    'gdn2': ('gdn2', 'chunk_gdn2'),
    'delta': ('delta', 'chunk_delta_rule'),
}


@dataclass(frozen=True)
class Selection:
    backend: str = 'original'
    strict: bool = True
    ops: tuple = tuple(OPERATORS)


_selection = ContextVar('rewy_amd_selection', default=Selection())
_counts = Counter()
_warned = set()


def record(op, event):
    _counts[f'{op}.{event}'] += 1


def stats(reset=False):
    result = dict(sorted(_counts.items()))
    if reset:
        _counts.clear()
    return result


def configure(backend='optimized', *, strict=True, ops=None):
    if backend not in ('original', 'optimized'):
        raise ValueError('backend must be original or optimized')
    ops = tuple(OPERATORS) if ops is None else tuple(ops)
    unknown = set(ops) - OPERATORS.keys()
    if unknown:
        raise ValueError(f'Unknown operators: {sorted(unknown)}')
    return _selection.set(Selection(backend, strict, ops))


@contextmanager
def use_backend(backend, *, strict=True, ops=None):
    token = configure(backend, strict=strict, ops=ops)
    try:
        yield
    finally:
        _selection.reset(token)


def source_fingerprint():
    """sha256 of every HIP source and header the library is built from."""
    root = Path(__file__).resolve().parent
    files = sorted((root / 'csrc').glob('*')) + sorted((root.parent / 'include').glob('*.h'))
    return {f.name: hashlib.sha256(f.read_bytes()).hexdigest() for f in files if f.is_file()}


@lru_cache(None)
def check_baseline():
    """Fail loudly when the HIP library is missing or older than its sources."""
    from .build import MANIFEST, OUT
    if not OUT.exists():
        raise RuntimeError(f'{OUT} is missing; build it with `python -m rewy_amd.build`.')
    if not MANIFEST.exists():
        raise RuntimeError(f'{MANIFEST} is missing; rebuild with `python -m rewy_amd.build`.')
    built = json.loads(MANIFEST.read_text())
    now = source_fingerprint()
    stale = sorted(n for n in set(now) | set(built['sources']) if now.get(n) != built['sources'].get(n))
    if stale:
        raise RuntimeError(f'librewy_hip.so is stale for {stale[:4]}; rebuild with `python -m rewy_amd.build`.')
    return built['arch']


@lru_cache(None)
def original_operator(op):
    family, name = OPERATORS[op]
    return getattr(importlib.import_module('rewy_amd.original_ops'), name)


def rejection_reason(op, arguments):
    """The release envelope is capability based, never benchmark-case based."""
    import torch
    q, k, v = (arguments.get(n) for n in ('q', 'k', 'v'))
    if not all(isinstance(x, torch.Tensor) and x.ndim == 4 for x in (q, k, v)):
        return 'expected rank-4 q/k/v'
    if q.device.type != 'cuda':
        return 'ROCm GPU required'
    if any(x.device != q.device for x in (k, v)):
        return 'mixed devices'
    if any(x.dtype != torch.bfloat16 for x in (q, k, v)):
        return 'release envelope uses BF16 q/k/v'
    if k.shape[-1] != 128 or v.shape[-1] != 128:
        return 'release envelope requires K=V=128'
    if q.shape != k.shape or k.shape[:3] != v.shape[:3]:
        return 'grouped heads or unequal q/k/v shapes'
    if arguments.get('cu_seqlens') is None and (k.shape[1] < 64 or k.shape[1] % 64):
        return 'sequence length must be a positive multiple of 64'
    if arguments.get('chunk_size', 64) != 64:
        return 'release envelope requires chunk_size=64'
    if arguments.get('cp_context') is not None:
        return 'context parallelism is not release-validated'
    if arguments.get('safe_gate', False):
        return 'safe_gate transform is not release-validated'
    if arguments.get('use_graph', False):
        return 'static variable-length graph buffers are not supported'
    if arguments.get('return_intermediate_states', False):
        return 'intermediate inference states are not supported'
    scale = arguments.get('scale')
    if scale is not None and scale != k.shape[-1] ** -.5:
        return 'custom scale is not release-validated'
    if op == 'gdn' and arguments.get('use_gate_in_kernel', False):
        return 'GDN fused gate is not release-validated'
    if op == 'gdn2' and arguments.get('use_gate_in_kernel', False):
        return 'GDN2 fused gate is not release-validated'
    if op == 'delta' and arguments.get('head_first', False):
        return 'head-first layout is not supported'
    return None


@lru_cache(None)
def optimized_operator(op):
    check_baseline()
    module = importlib.import_module(f'rewy_amd._compat.{op}')
    return getattr(module, OPERATORS[op][1])


@lru_cache(None)
def operator(op):
    if op not in OPERATORS:
        raise ValueError(f'Unknown operator {op!r}')
    base = original_operator(op)
    signature = inspect.signature(base)

    @wraps(base)
    def call(*args, **kwargs):
        config = _selection.get()
        if config.backend == 'original' or op not in config.ops:
            record(op, 'original_forward')
            return base(*args, **kwargs)
        bound = signature.bind(*args, **kwargs)
        bound.apply_defaults()
        arguments = dict(bound.arguments)
        arguments.update(arguments.pop('kwargs', {}))
        reason = rejection_reason(op, arguments)
        if reason:
            record(op, 'rejected:' + reason)
            if config.strict:
                raise RuntimeError(f'rewy_amd {op}: {reason}')
            key = (op, reason)
            if key not in _warned:
                warnings.warn(f'rewy_amd {op} using original: {reason}', RuntimeWarning, stacklevel=2)
                _warned.add(key)
            record(op, 'fallback_forward')
            return base(*args, **kwargs)
        result = optimized_operator(op)(*args, **kwargs)
        record(op, 'optimized_forward')
        return result
    return call


def assert_used(ops=None, *, backward=True):
    ops = _selection.get().ops if ops is None else ops
    suffix = 'optimized_backward' if backward else 'optimized_forward'
    missing = [op for op in ops if not _counts.get(f'{op}.{suffix}', 0)]
    if missing:
        raise RuntimeError(f'No {suffix} calls for {missing}; check integration and whether backward ran.')
