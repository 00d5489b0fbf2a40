"""Import-path twin of the reference's `fast_delta_rule._compat.gdn` (reference
src/fast_delta_rule/_compat/gdn.py:271): ``chunk_gated_delta_rule`` bound to the optimized (HIP) backward."""
from .api import make_gdn

chunk_gated_delta_rule = make_gdn("optimized")
chunk_gdn = chunk_gated_delta_rule      # (reference _compat/gdn.py:470)
