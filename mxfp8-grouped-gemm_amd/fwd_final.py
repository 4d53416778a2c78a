"""Reference-compatible module name: ``from fwd_final import fwd_ge``
(fwd_final.py:121-131 in the reference), backed by libmxgg.so."""
from mxfp8gg.ops import fwd_ge

__all__ = ["fwd_ge"]
