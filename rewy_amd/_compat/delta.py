"""Import-path twin of the reference's `fast_delta_rule._compat.delta` (reference
src/fast_delta_rule/_compat/delta.py:144): ``chunk_delta_rule`` bound to the optimized (HIP) backward."""
from .api import make_delta

chunk_delta_rule = make_delta("optimized")
