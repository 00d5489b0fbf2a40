"""MI355X-native chunked delta-rule backward (DeltaNet, GDN, KDA, GDN2).

Same public surface as the reference package ``fast_delta_rule``
(reference src/fast_delta_rule/__init__.py:1-40): ``enable``, ``disable``,
``use_backend``, ``stats``, ``assert_used`` and the four ``chunk_*`` operators
routed by the active backend.  Importing the package imports no torch and
loads no library.
"""
from .runtime import use_backend, stats, assert_used

__version__ = '0.1.0'


def enable(backend='optimized', *, strict=True, ops=None, integrations=()):
    """Select the backend for subsequent forwards.  The reference's FLA and
    model integrations (integrations/fla.py, integrations/models.py) have no
    counterpart here: the ``chunk_*`` functions below are the entry points."""
    from .runtime import configure, check_baseline
    if backend == 'optimized':
        check_baseline()
    for name in integrations:
        raise ValueError(f'Unknown integration: {name}')
    configure(backend, strict=strict, ops=ops)


def disable():
    from .runtime import configure
    configure('original')


def chunk_kda(*args, **kwargs):
    from .runtime import operator
    return operator('kda')(*args, **kwargs)


def chunk_gated_delta_rule(*args, **kwargs):
    from .runtime import operator
    return operator('gdn')(*args, **kwargs)


def chunk_gdn2(*args, **kwargs):
    from .runtime import operator
    return operator('gdn2')(*args, **kwargs)


def chunk_delta_rule(*args, **kwargs):
    from .runtime import operator
    return operator('delta')(*args, **kwargs)
