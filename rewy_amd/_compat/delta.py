"""chunk_delta_rule whose backward runs on the gfx950 HIP kernels (reference _compat/delta.py)."""
from .api import ChunkFunction, make_delta

chunk_delta_rule = make_delta("optimized")

__all__ = ["chunk_delta_rule", "ChunkFunction"]
