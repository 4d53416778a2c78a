"""Autograd wrapper: the MXFP8 grouped GEMM as a differentiable torch op.

The reference trains through torchao's MXFP8 grouped-mm autograd function
(swapped in by patch_kernels.py:15-48 and the converter that port_mxfp8.py
writes into torchtitan, port_mxfp8.py:200-218, 317-336); torchao itself is not
part of the reference.  This module provides the same operation on this
library's kernels:

  forward  : y[rows of g] = x[rows of g] . W[g]^T      (x, W cast along K)
  backward : dx = dy . W  per group                   (dy, W cast along N)
             dW[g] = dy_g^T . x_g                     (dy, x cast along tokens)

Weights use the torchtitan GroupedExperts layout W [E, out, in].  Groups may
be ragged or empty and need no padding: the token-axis casts pad each group
to 32 internally.  All casts use the same E8M0 rule (RCEIL by default, the
reference's recipe "mxfp8_rceil", port_mxfp8.py:207-213).
"""
from __future__ import annotations

import torch

from . import ops


class MXFP8GroupedMM(torch.autograd.Function):
    """y = grouped x . W^T with MXFP8 operands and fp32 accumulation."""

    @staticmethod
    def forward(ctx, x, w, offs, scaling_mode="rceil"):
        if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
            raise TypeError("x and w must be bfloat16")
        offs = ops._group_ends(offs, w.shape[0], x.device)
        xq, xs = ops.to_mxfp8_dim0(x, scaling_mode)
        wq, ws = ops.to_mxfp8_dim0(w, scaling_mode)
        y = ops.grouped_mm(xq, wq, offs, xs, ws, out_dtype=torch.bfloat16)
        ctx.save_for_backward(x, w, offs)
        ctx.scaling_mode = scaling_mode
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, offs = ctx.saved_tensors
        mode = ctx.scaling_mode
        dy = dy.to(torch.bfloat16)
        if dy.stride(-1) != 1:
            dy = dy.contiguous()
        dx = dw = None
        if ctx.needs_input_grad[0]:
            dx = ops.grouped_dgrad(dy, w, offs, scaling_mode=mode)
        if ctx.needs_input_grad[1]:
            go, gos, pad = ops.to_mxfp8_dim1(dy, offs, mode)
            ia, ias, _ = ops.to_mxfp8_dim1(x, offs, mode)
            dw = ops.grouped_wgrad(go, ia, pad, gos, ias, out_dtype=w.dtype)
        return dx, dw, None, None


def mxfp8_grouped_mm(x: torch.Tensor, w: torch.Tensor, offs: torch.Tensor,
                     scaling_mode: str = "rceil") -> torch.Tensor:
    """Differentiable MXFP8 grouped GEMM: x bf16 [M, K], w bf16 [E, N, K],
    offs int32 group ends [E] (or [E+1] with a leading 0) -> bf16 [M, N].
    Rows after the last group end are left unwritten, as in the forward op."""
    return MXFP8GroupedMM.apply(x, w, offs, scaling_mode)


def moe_ffn(x: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor,
            offs: torch.Tensor, scaling_mode: str = "rceil") -> torch.Tensor:
    """One DeepSeek-V3-style expert FFN over routed tokens (the layer step of
    the reference's e2e_bench.py:56-134): gate+up projection with the fused
    weight w_gate_up [E, 2F, H] (gate rows first), SiLU(gate) * up, down
    projection w_down [E, H, F]."""
    h = mxfp8_grouped_mm(x, w_gate_up, offs, scaling_mode)
    f = w_down.shape[2]
    a = torch.nn.functional.silu(h[:, :f]) * h[:, f:]
    return mxfp8_grouped_mm(a, w_down, offs, scaling_mode)
