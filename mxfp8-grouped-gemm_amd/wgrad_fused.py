"""Reference-compatible module name for the wgrad entry points
(wgrad_fused.py:22-112 in the reference), backed by libmxgg.so."""
from mxfp8gg.ops import _best_config, wgrad_fused, wgrad_kernel, wgrad_prepare

__all__ = ["_best_config", "wgrad_fused", "wgrad_prepare", "wgrad_kernel"]
