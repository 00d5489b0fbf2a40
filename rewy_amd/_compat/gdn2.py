"""chunk_gdn2 whose backward runs on the gfx950 HIP kernels (reference _compat/gdn2.py)."""
from .api import ChunkFunction, make_gdn2

chunk_gdn2 = make_gdn2("optimized")

__all__ = ["chunk_gdn2", "ChunkFunction"]
