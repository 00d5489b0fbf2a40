"""chunk_gated_delta_rule whose backward runs on the gfx950 HIP kernels (reference _compat/gdn.py)."""
from .api import ChunkFunction, make_gdn

chunk_gated_delta_rule = make_gdn("optimized")

__all__ = ["chunk_gated_delta_rule", "ChunkFunction"]
