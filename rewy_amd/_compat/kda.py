"""Import-path twin of the reference's `fast_delta_rule._compat.kda` (reference
src/fast_delta_rule/_compat/kda.py:214): ``chunk_kda`` bound to the optimized (HIP) backward."""
from .api import make_kda

chunk_kda = make_kda("optimized")
