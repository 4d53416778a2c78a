"""Reference-compatible module name: ``from fused_fwd import fused_grouped_fwd``.

Same entry point as the reference's fused_fwd.py:172-229, backed by the gfx950
HIP kernel in libmxgg.so (no Triton).
"""
from mxfp8gg.ops import fused_grouped_fwd

__all__ = ["fused_grouped_fwd"]
