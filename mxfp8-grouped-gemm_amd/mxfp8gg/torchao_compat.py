"""Swap-in surface for an MoE trainer built on torchao's ROCm MXFP8 path.

The reference replaces attributes of
``torchao.prototype.moe_training.kernels.mxfp8.rocm_mxfp8_mm``
(patch_kernels.py:25-35, port_mxfp8.py:333-336) and the trainer quantises
with ``triton_to_mxfp8_dim0 / dim1`` (port_mxfp8.py:43; memory/2026-06-09.md:20).
Those functions live in an external torchao fork whose exact signatures are
not in the reference, so the signatures below are this library's own,
documented choice (same names, same argument meaning as the torchao quant
helpers and torch._scaled_grouped_mm).
"""
from __future__ import annotations

import torch

from . import ops

_E8M0 = getattr(torch, "float8_e8m0fnu", None)


def _e8m0_view(s: torch.Tensor) -> torch.Tensor:
    return s.view(_E8M0) if _E8M0 is not None else s


def triton_to_mxfp8_dim0(x: torch.Tensor, inner_block_size: int = 32, scaling_mode="floor",
                         scale_layout: str = "row"):
    """torchao-named row-wise cast: returns (data e4m3 like x, scales e8m0 [..., K/32]).

    The scales are contiguous (scale_layout "row", as torchao returns them:
    .view() and reshape work); a grouped GEMM call then re-lays them
    block-major on the device (1/32 of the payload's bytes).  "block" returns
    the block-major view the GEMM reads in place."""
    if inner_block_size != 32:
        raise ValueError("only 32-element blocks are supported (MX block size)")
    q, s = ops.to_mxfp8_dim0(x, scaling_mode, scale_layout)
    return q, _e8m0_view(s)


def triton_to_mxfp8_dim1(x: torch.Tensor, inner_block_size: int = 32, scaling_mode="floor",
                         scale_layout: str = "row"):
    """torchao-named column-wise cast of a row-major [M, K] tensor.

    Returns (data, scales): data is the [M, K] logical view of column-major
    storage (a [K, M] row-major buffer transposed), scales e8m0 [K, M/32],
    contiguous (scale_layout "row"; "block" as in triton_to_mxfp8_dim0).
    M must be a multiple of 32 (no grouping: one block sequence per column).
    """
    if inner_block_size != 32:
        raise ValueError("only 32-element blocks are supported (MX block size)")
    x2 = x.reshape(-1, x.shape[-1])
    M = x2.shape[0]
    if M % 32 != 0:
        raise ValueError(f"dim1 cast needs rows % 32 == 0, got {M}")
    qt, st, _ = ops.to_mxfp8_dim1(x2, None, scaling_mode, scale_layout)
    return qt.t(), _e8m0_view(st)


def triton_mxfp8_grouped_mm(A_data, B_data, A_scale, B_scale, offs, out_dtype=torch.bfloat16,
                            **kwargs):
    """Forward grouped GEMM with MXFP8 operands.

    A_data [M, K] e4m3, A_scale [M, K/32]; B_data the experts either as
    [E, N, K] (K contiguous) or as its transposed view [E, K, N] (the B_t
    operand of torch._scaled_grouped_mm); B_scale [E, N, K/32] unswizzled;
    offs [E] int32 cumulative token ends.  Extra keyword arguments (e.g.
    ``ctas_per_cu``, dropped by the reference's wrapper at port_mxfp8.py:325-332)
    are ignored.
    """
    del kwargs
    w = B_data
    if w.dim() == 3 and w.stride(-1) != 1 and w.stride(-2) == 1:
        w = w.transpose(-2, -1)  # [E, K, N] view of [E, N, K] storage
    return ops.grouped_mm(A_data, w, offs, A_scale, B_scale, out_dtype=out_dtype)


def triton_mxfp8_wgrad(grad_out_t, grad_out_t_scale, input_t, input_t_scale, offs,
                       out_dtype=torch.float32, **kwargs):
    """Weight gradient dW[g] = dY_g^T X_g from token-contiguous operands.

    grad_out_t [N, M] e4m3 + [N, M/32]; input_t [K, M] e4m3 + [K, M/32];
    offs [E] int32 token ends (multiples of 32).  Returns [E, N, K].
    """
    del kwargs
    return ops.grouped_wgrad(grad_out_t, input_t, offs, grad_out_t_scale, input_t_scale,
                             out_dtype=out_dtype)


# The reference routes both wgrad names to the same kernel (patch_kernels.py:28-31).
triton_mxfp8_wgrad_v2 = triton_mxfp8_wgrad


def apply(target=None, verbose: bool = True):
    """Swap this library's kernels into torchao's ROCm MXFP8 module.

    Mirrors patch_kernels.apply() (patch_kernels.py:15-48): replaces
    triton_mxfp8_grouped_mm / triton_mxfp8_wgrad / triton_mxfp8_wgrad_v2,
    re-binds the package attribute rocm_mxfp8_mm, patches the quant helpers
    when the quant module is importable, and verifies the swap.  `target`
    overrides the module to patch (used by tests; torchao is not a dependency).
    """
    import importlib
    import sys

    if target is None:
        target = importlib.import_module(
            "torchao.prototype.moe_training.kernels.mxfp8.rocm_mxfp8_mm")
    target.triton_mxfp8_grouped_mm = triton_mxfp8_grouped_mm
    target.triton_mxfp8_wgrad = triton_mxfp8_wgrad
    target.triton_mxfp8_wgrad_v2 = triton_mxfp8_wgrad_v2
    pkg_name = target.__name__.rpartition(".")[0]
    pkg = sys.modules.get(pkg_name)
    if pkg is not None:
        pkg.rocm_mxfp8_mm = target
    quant = sys.modules.get(pkg_name + ".quant")
    if quant is None:
        try:
            quant = importlib.import_module(pkg_name + ".quant")
        except ImportError:
            quant = None
    if quant is not None:
        quant.triton_to_mxfp8_dim0 = triton_to_mxfp8_dim0
        quant.triton_to_mxfp8_dim1 = triton_to_mxfp8_dim1
    mod = sys.modules[target.__name__] if target.__name__ in sys.modules else target
    assert mod.triton_mxfp8_grouped_mm is triton_mxfp8_grouped_mm, "Forward patch failed!"
    assert mod.triton_mxfp8_wgrad is triton_mxfp8_wgrad, "Backward patch failed!"
    if verbose:
        print("[mxfp8gg] swapped gfx950 MXFP8 grouped GEMM kernels into " + target.__name__)
    return target
