"""chunk_kda whose backward runs on the gfx950 HIP kernels (reference _compat/kda.py)."""
from .api import ChunkFunction, make_kda

chunk_kda = make_kda("optimized")

__all__ = ["chunk_kda", "ChunkFunction"]
