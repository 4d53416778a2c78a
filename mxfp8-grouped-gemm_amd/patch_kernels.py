"""Reference-compatible ``patch_kernels.apply()`` (patch_kernels.py:15-48 in the
reference): swaps this library's kernels into torchao's rocm_mxfp8_mm module.

Usage: import and call apply() before the trainer imports torchao's MoE path.
"""
from mxfp8gg.torchao_compat import apply

__all__ = ["apply"]

if __name__ == "__main__":
    apply()
