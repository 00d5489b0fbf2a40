"""The four operators with the original (7-product, PyTorch) backward.

These play the role of FLA's unpatched operators in the reference
(``runtime.original_operator``, reference runtime.py:69-73): the ``original``
backend, the non-strict fallback, and the same-GPU comparator.  They accept any
sequence length (zero-padded to a multiple of 64 internally).
"""
from ._compat.api import make_delta, make_gdn, make_gdn2, make_kda

chunk_kda = make_kda("original")
chunk_gated_delta_rule = make_gdn("original")
chunk_gdn2 = make_gdn2("original")
chunk_delta_rule = make_delta("original")
