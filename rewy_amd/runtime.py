"""Backend routing, the release envelope and the dispatch report.

Public behaviour follows reference ``src/fast_delta_rule/runtime.py``: the
operator names (:14-19), a context-local backend selection (:21-27),
``family.event`` counters (:31-37), ``configure`` / ``use_backend`` (:39-50),
the envelope's rejection messages (:75-106), strict-raise or warn-and-fall-back
routing (:114-143) and ``assert_used`` (:145-149).  Importing this module
imports no torch.

The implementation is this package's own: the envelope is an ordered table of
``Rule`` objects evaluated by ``rejection_reason``, and a ``Dispatcher`` per
operator owns its original/optimized implementations and its counters.
Where the platform forces a difference:

* ``original`` is this package's PyTorch restatement of the original
  7-product formulation (``rewy_amd.original``) instead of FLA;
* ``check_baseline`` fingerprints this package's HIP library against the
  sources it was built from (the reference seals FLA's sources, :52-67);
* packed variable-length batches (``cu_seqlens``) are accepted: every kernel takes
  the batch's chunk map, sequences starting anywhere (the reference rejects them);
* grouped value heads (HV a multiple of H) are accepted for KDA, GDN and DeltaNet:
  the kernels map value heads to q / k heads themselves (the reference rejects them).
"""
from collections import Counter
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass, field
from functools import lru_cache, update_wrapper
import hashlib
import inspect
import json
from pathlib import Path
import warnings

# public family key -> (reference module family, public function name)
OPERATORS = {
    'kda': ('kda', 'chunk_kda'),
    'gdn': ('gdn', 'chunk_gated_delta_rule'),
    'gdn2': ('gdn2', 'chunk_gdn2'),
    'delta': ('delta', 'chunk_delta_rule'),
}

# public function name -> factory in rewy_amd._compat.api
_FACTORIES = {'kda': 'make_kda', 'gdn': 'make_gdn', 'gdn2': 'make_gdn2', 'delta': 'make_delta'}


@dataclass(frozen=True)
class Selection:
    """The active choice: backend, strictness and the operators it covers."""
    backend: str = 'original'
    strict: bool = True
    ops: tuple = tuple(OPERATORS)

    def routes(self, op):
        return self.backend == 'optimized' and op in self.ops


_selection = ContextVar('rewy_amd_selection', default=Selection())


class _Report:
    """Process-global event counts (``<op>.<event>``) and the warn-once set."""

    def __init__(self):
        self.counts = Counter()
        self.warned = set()

    def bump(self, op, event):
        self.counts['.'.join((op, event))] += 1

    def snapshot(self, reset):
        out = {key: self.counts[key] for key in sorted(self.counts)}
        if reset:
            self.counts.clear()
        return out

    def warn_once(self, op, reason):
        if (op, reason) in self.warned:
            return
        self.warned.add((op, reason))
        warnings.warn(f'rewy_amd {op} using original: {reason}', RuntimeWarning, stacklevel=4)


_report = _Report()


def record(op, event):
    _report.bump(op, event)


def stats(reset=False):
    return _report.snapshot(reset)


def configure(backend='optimized', *, strict=True, ops=None):
    if backend not in ('original', 'optimized'):
        raise ValueError('backend must be original or optimized')
    chosen = tuple(OPERATORS if ops is None else ops)
    unknown = sorted(set(chosen).difference(OPERATORS))
    if unknown:
        raise ValueError(f'Unknown operators: {unknown}')
    return _selection.set(Selection(backend=backend, strict=strict, ops=chosen))


@contextmanager
def use_backend(backend, *, strict=True, ops=None):
    token = configure(backend, strict=strict, ops=ops)
    try:
        yield
    finally:
        _selection.reset(token)


def source_fingerprint():
    """sha256 of every HIP source and header the library is built from."""
    pkg = Path(__file__).resolve().parent
    inputs = [p for p in sorted((pkg / 'csrc').glob('*')) + sorted((pkg.parent / 'include').glob('*.h'))
              if p.is_file()]
    return {p.name: hashlib.sha256(p.read_bytes()).hexdigest() for p in inputs}


@lru_cache(None)
def check_baseline():
    """Fail loudly when the HIP library is missing or older than its sources."""
    from .build import MANIFEST, OUT
    hint = 'build it with `python -m rewy_amd.build`.'
    for path in (OUT, MANIFEST):
        if not path.exists():
            raise RuntimeError(f'{path} is missing; {hint}')
    manifest = json.loads(MANIFEST.read_text())
    current, built = source_fingerprint(), manifest['sources']
    changed = sorted(name for name in current.keys() | built.keys() if current.get(name) != built.get(name))
    if changed:
        raise RuntimeError(f'librewy_hip.so is stale for {changed[:4]}; rebuild with `python -m rewy_amd.build`.')
    return manifest['arch']


# --------------------------------------------------------------------------
# The release envelope: capability based, never benchmark-case based.
# --------------------------------------------------------------------------

@dataclass(frozen=True)
class Rule:
    """One envelope condition: ``rejects(op, args)`` true -> ``message``."""
    message: str
    rejects: object
    ops: tuple = field(default=tuple(OPERATORS))


def _qkv(args):
    return args.get('q'), args.get('k'), args.get('v')


def _not_rank4(torch, args):
    return not all(isinstance(t, torch.Tensor) and t.ndim == 4 for t in _qkv(args))


# grouped value heads (HV a multiple of H) run natively for the families whose
# reference operators define them (KDA, GDN; DeltaNet's kernels are GDN's without a gate)
_GROUPED_OK = ('kda', 'gdn', 'delta')


def _bad_heads(args):
    q, k, v = _qkv(args)
    if q.shape != k.shape or k.shape[:2] != v.shape[:2]:
        return True
    H, HV = k.shape[2], v.shape[2]
    if HV == H:
        return False
    return args.get('_op') not in _GROUPED_OK or HV % H != 0


def _bad_length(torch, args):
    if args.get('cu_seqlens') is not None:
        return False
    T = args['k'].shape[1]
    return T < 64 or T % 64 != 0


def _bad_scale(torch, args):
    s = args.get('scale')
    return s is not None and s != args['k'].shape[-1] ** -0.5


_ENVELOPE = (
    Rule('expected rank-4 q/k/v', _not_rank4),
    Rule('ROCm GPU required', lambda torch, a: a['q'].device.type != 'cuda'),
    Rule('mixed devices', lambda torch, a: a['k'].device != a['q'].device or a['v'].device != a['q'].device),
    Rule('release envelope uses BF16 q/k/v', lambda torch, a: any(t.dtype != torch.bfloat16 for t in _qkv(a))),
    Rule('release envelope requires K=V=128', lambda torch, a: (a['k'].shape[-1], a['v'].shape[-1]) != (128, 128)),
    Rule('grouped heads or unequal q/k/v shapes', lambda torch, a: _bad_heads(a)),
    Rule('sequence length must be a positive multiple of 64', _bad_length),
    Rule('release envelope requires chunk_size=64', lambda torch, a: a.get('chunk_size', 64) != 64),
    Rule('context parallelism is not release-validated', lambda torch, a: a.get('cp_context') is not None),
    Rule('safe_gate transform is not release-validated', lambda torch, a: bool(a.get('safe_gate', False))),
    Rule('static variable-length graph buffers are not supported', lambda torch, a: bool(a.get('use_graph', False))),
    Rule('intermediate inference states are not supported',
         lambda torch, a: bool(a.get('return_intermediate_states', False))),
    Rule('custom scale is not release-validated', _bad_scale),
    Rule('GDN fused gate is not release-validated', lambda torch, a: bool(a.get('use_gate_in_kernel', False)),
         ops=('gdn',)),
    Rule('GDN2 fused gate is not release-validated', lambda torch, a: bool(a.get('use_gate_in_kernel', False)),
         ops=('gdn2',)),
    Rule('head-first layout is not supported', lambda torch, a: bool(a.get('head_first', False)), ops=('delta',)),
)


def rejection_reason(op, arguments):
    """The first envelope rule the call breaks, or None when it is accepted."""
    import torch
    arguments = dict(arguments, _op=op)
    for rule in _ENVELOPE:
        if op in rule.ops and rule.rejects(torch, arguments):
            return rule.message
    return None


# --------------------------------------------------------------------------
# Routing
# --------------------------------------------------------------------------

def _implementation(op, backend):
    from ._compat import api
    return getattr(api, _FACTORIES[op])(backend)


@lru_cache(None)
def original_operator(op):
    return _implementation(op, 'original')


@lru_cache(None)
def optimized_operator(op):
    check_baseline()
    return _implementation(op, 'optimized')


class Dispatcher:
    """The public callable of one operator.  Each call reads the active
    Selection, screens optimized calls through the envelope, and either runs
    the optimized implementation, raises (strict), or falls back to the
    original one with a warning; every outcome is counted."""

    def __init__(self, op):
        self.op = op
        self.original = original_operator(op)
        self.signature = inspect.signature(self.original)
        update_wrapper(self, self.original)

    def arguments(self, args, kwargs):
        bound = self.signature.bind(*args, **kwargs)
        bound.apply_defaults()
        named = dict(bound.arguments)
        named.update(named.pop('kwargs', {}))   # A_log, dt_bias and legacy options
        return named

    def __call__(self, *args, **kwargs):
        selection = _selection.get()
        if not selection.routes(self.op):
            record(self.op, 'original_forward')
            return self.original(*args, **kwargs)
        reason = rejection_reason(self.op, self.arguments(args, kwargs))
        if reason is None:
            out = optimized_operator(self.op)(*args, **kwargs)
            record(self.op, 'optimized_forward')
            return out
        record(self.op, 'rejected:' + reason)
        if selection.strict:
            raise RuntimeError(f'rewy_amd {self.op}: {reason}')
        _report.warn_once(self.op, reason)
        record(self.op, 'fallback_forward')
        return self.original(*args, **kwargs)


@lru_cache(None)
def operator(op):
    if op not in OPERATORS:
        raise ValueError(f'Unknown operator {op!r}')
    return Dispatcher(op)


def assert_used(ops=None, *, backward=True):
    wanted = _selection.get().ops if ops is None else ops
    event = 'optimized_backward' if backward else 'optimized_forward'
    counts = _report.counts
    missing = [op for op in wanted if counts.get(f'{op}.{event}', 0) == 0]
    if missing:
        raise RuntimeError(f'No {event} calls for {missing}; check integration and whether backward ran.')
