"""Import-path twin of the reference's `fast_delta_rule._compat.gdn2` (reference
src/fast_delta_rule/_compat/gdn2.py:204): ``chunk_gdn2`` bound to the optimized (HIP) backward."""
from .api import make_gdn2

chunk_gdn2 = make_gdn2("optimized")
