"""Token routing around the expert GEMMs of a top-k MoE layer (one GPU).

The reference's trainer takes dispatch and combine from torchtitan's token
dispatcher, swapped in with ``pad_multiple=32`` (port_mxfp8.py:214, 240):
the (token, k) slots are sorted by expert with a stable argsort, the routed
input is ``x[sorted_slots // topk]`` with every expert's rows padded to a
multiple of 32, and the experts' output is scaled by the routing score and
scattered back to token order.  Here the plan is computed on the device by
three small kernels (no host sync), the gather is fused into the MXFP8 casts of the expert
input (the bf16 routed copy is never written), and the combine sums the top-k
terms in fp32 and rounds once.

    plan = route_plan(expert_idx, num_experts)          # [T, topk] int
    q, s, qt, st, pad = gather_to_mxfp8_dual(x, plan)   # routed MXFP8 input
    ...                                                  # grouped GEMMs over plan.offs
    out = combine(y_routed, plan, scores)                # [T, H] bf16

Expert-parallel all-to-all (several GPUs) is not part of this module: with
one GPU every expert is local and dispatch is this gather.
"""
from __future__ import annotations

from typing import NamedTuple

import torch

from . import _lib, ops
from .ops import (_FP8, _block_major_buffer, _mode, _need_gpu, _stream_ptr,
                  padded_token_capacity)

__all__ = ["RoutePlan", "route_plan", "gather_rows", "gather_to_mxfp8_dual",
           "gather_to_mxfp8_dim0", "combine", "combine_score_grad"]


class RoutePlan(NamedTuple):
    """Device-side dispatch plan of one routing decision.

    perm   int32 [tokens * topk]  routed row of each slot s = t * topk + k (-1: dropped)
    src    int32 [rows]           slot held by each routed row (-1: padding)
    offs   int32 [E]              cumulative padded group ends (the GEMMs' group ends)
    counts int32 [E]              slots routed to each expert
    """
    perm: torch.Tensor
    src: torch.Tensor
    offs: torch.Tensor
    counts: torch.Tensor
    tokens: int
    topk: int
    num_experts: int
    pad_multiple: int

    @property
    def rows(self) -> int:
        """Rows of the routed layout (a capacity: rows past offs[-1] are empty)."""
        return self.src.numel()


# Routings of at most this many slots take the one-workgroup plan (a single
# launch); larger ones the plan over one workgroup per 4096 slots.
_PLAN_ONE_WORKGROUP_SLOTS = 4096


def route_plan(expert_idx: torch.Tensor, num_experts: int, pad_multiple: int = 32) -> RoutePlan:
    """Sort the slots of ``expert_idx`` ([tokens, topk] integer expert ids on the
    GPU) by expert, stably, each expert's rows padded to ``pad_multiple``.
    Ids outside [0, num_experts) drop their slot.  The routed layout gets
    ``tokens * topk + num_experts * (pad_multiple - 1)`` rows, enough for any
    routing, so nothing is read back to size it."""
    _need_gpu(expert_idx, "expert_idx")
    if expert_idx.dim() == 1:
        expert_idx = expert_idx[:, None]
    if expert_idx.dim() != 2 or expert_idx.dtype not in (torch.int32, torch.int64):
        raise TypeError("expert_idx must be an integer tensor [tokens, topk]")
    T, K = expert_idx.shape
    idx = expert_idx.to(torch.int32).contiguous()
    rows = T * K + num_experts * (pad_multiple - 1)
    dev = expert_idx.device
    perm = torch.empty(T * K, dtype=torch.int32, device=dev)
    src = torch.empty(rows, dtype=torch.int32, device=dev)
    offs = torch.empty(num_experts, dtype=torch.int32, device=dev)
    counts = torch.empty(num_experts, dtype=torch.int32, device=dev)
    lib = _lib.load()
    if T * K <= _PLAN_ONE_WORKGROUP_SLOTS:
        # one workgroup's worth of slots: one launch, no workspace
        _lib.check(
            lib.mxgg_route_plan(idx.data_ptr(), T, K, num_experts, pad_multiple, rows,
                                perm.data_ptr(), src.data_ptr(), offs.data_ptr(),
                                counts.data_ptr(), _stream_ptr(idx)),
            "route_plan",
        )
    else:
        # the many-workgroup form (one workgroup per 4096 slots); its
        # workspace holds a count per (workgroup, expert)
        nbytes = int(lib.mxgg_route_plan_workspace_bytes(T, K, num_experts))
        if nbytes < 0:
            raise ValueError(f"route_plan: invalid shape tokens={T}, topk={K}, "
                             f"experts={num_experts}")
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        _lib.check(
            lib.mxgg_route_plan_ws(idx.data_ptr(), T, K, num_experts, pad_multiple, rows,
                                   perm.data_ptr(), src.data_ptr(), offs.data_ptr(),
                                   counts.data_ptr(), ws.data_ptr(), nbytes, _stream_ptr(idx)),
            "route_plan",
        )
    return RoutePlan(perm, src, ops._mark_ends(offs), counts, T, K, num_experts, pad_multiple)


def _rows_ok(t: torch.Tensor) -> torch.Tensor:
    if t.stride(-1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0:
        return t
    return t.contiguous()


def _scores(scores, plan: RoutePlan, device):
    if scores is None:
        return None
    _need_gpu(scores, "scores")
    if scores.numel() != plan.tokens * plan.topk:
        raise ValueError(f"scores must have tokens * topk = {plan.tokens * plan.topk} elements")
    return scores.to(torch.float32).contiguous()


def gather_rows(x: torch.Tensor, plan: RoutePlan, row_scale: torch.Tensor | None = None):
    """The routed input in bf16: row r = x[src[r] // topk] (zero for padding),
    times row_scale[src[r]] rounded to bf16 when given.  [plan.rows, H]."""
    _need_gpu(x, "x")
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] % 8 != 0:
        raise TypeError("x must be a 2-D bfloat16 tensor [tokens, H] with H % 8 == 0")
    x2 = _rows_ok(x)
    sc = _scores(row_scale, plan, x.device)
    out = torch.empty((plan.rows, x.shape[1]), dtype=torch.bfloat16, device=x.device)
    lib = _lib.load()
    _lib.check(
        lib.mxgg_gather_rows(x2.data_ptr(), x2.shape[0], x2.shape[1], x2.stride(0),
                             plan.src.data_ptr(), plan.topk,
                             sc.data_ptr() if sc is not None else None, plan.rows,
                             out.data_ptr(), out.stride(0), _stream_ptr(x)),
        "gather_rows",
    )
    return out


def gather_to_mxfp8_dual(x: torch.Tensor, plan: RoutePlan, scaling_mode="rceil",
                         row_scale: torch.Tensor | None = None):
    """Both MXFP8 casts of the routed rows (gather_rows(x, plan, row_scale)),
    read straight from token order.  Returns (q, s, qt, st, offs_pad) like
    to_mxfp8_dual(gather_rows(x, plan, row_scale), plan.offs)."""
    _need_gpu(x, "x")
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] % 32 != 0:
        raise TypeError("x must be a 2-D bfloat16 tensor [tokens, H] with H % 32 == 0")
    x2 = _rows_ok(x)
    sc = _scores(row_scale, plan, x.device)
    M, C, E = plan.rows, x.shape[1], plan.num_experts
    cap = padded_token_capacity(M, E)
    dev = x.device
    q = torch.empty((M, C), dtype=_FP8, device=dev)
    sbuf = _block_major_buffer(M, C // 32, dev)
    qt = torch.empty((C, cap), dtype=_FP8, device=dev)
    stbuf = _block_major_buffer(C, cap // 32, dev)
    ends_pad = torch.empty(E, dtype=torch.int32, device=dev)
    lib = _lib.load()
    _lib.check(
        lib.mxgg_gather_quant_dual(
            x2.data_ptr(), x2.shape[0], C, x2.stride(0), plan.src.data_ptr(), plan.topk,
            sc.data_ptr() if sc is not None else None, M, plan.offs.data_ptr(), E, cap,
            q.data_ptr(), C, sbuf.data_ptr(), sbuf.stride(0), qt.data_ptr(), cap,
            stbuf.data_ptr(), stbuf.stride(0), _lib.SCALES_BLOCK_MAJOR, ends_pad.data_ptr(),
            _mode(scaling_mode), _stream_ptr(x)),
        "gather_quant_dual",
    )
    return q, sbuf[:, :M].t(), qt, stbuf[:, :C].t(), ends_pad


def gather_to_mxfp8_dim0(x: torch.Tensor, plan: RoutePlan, scaling_mode="rceil"):
    """The row-wise MXFP8 cast of the routed rows (gather_rows(x, plan)), read
    straight from token order: the expert input of a forward-only pass.
    Returns (q [plan.rows, H], s) like to_mxfp8_dim0(gather_rows(x, plan))."""
    _need_gpu(x, "x")
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] % 32 != 0:
        raise TypeError("x must be a 2-D bfloat16 tensor [tokens, H] with H % 32 == 0")
    x2 = _rows_ok(x)
    M, C = plan.rows, x.shape[1]
    q = torch.empty((M, C), dtype=_FP8, device=x.device)
    sbuf = _block_major_buffer(M, C // 32, x.device)
    lib = _lib.load()
    _lib.check(
        lib.mxgg_gather_quant_dim0(
            x2.data_ptr(), x2.shape[0], C, x2.stride(0), plan.src.data_ptr(), plan.topk, M,
            q.data_ptr(), C, sbuf.data_ptr(), sbuf.stride(0), _lib.SCALES_BLOCK_MAJOR,
            _mode(scaling_mode), _stream_ptr(x)),
        "gather_quant_dim0",
    )
    return q, sbuf[:, :M].t()


def combine(y: torch.Tensor, plan: RoutePlan, scores: torch.Tensor | None = None):
    """Back to token order: out[t] = bf16(sum_k bf16(y[perm[t, k]] * scores[t, k]))
    with the sum in fp32 in k order; without scores the plain sum of the
    routed rows (the input gradient of the gather).  y: bf16 [plan.rows, H]."""
    _need_gpu(y, "y")
    if y.dtype != torch.bfloat16 or y.dim() != 2 or y.shape[1] % 8 != 0:
        raise TypeError("y must be a 2-D bfloat16 tensor [rows, H] with H % 8 == 0")
    y2 = _rows_ok(y)
    sc = _scores(scores, plan, y.device)
    out = torch.empty((plan.tokens, y.shape[1]), dtype=torch.bfloat16, device=y.device)
    lib = _lib.load()
    _lib.check(
        lib.mxgg_combine(y2.data_ptr(), y2.shape[0], y2.shape[1], y2.stride(0),
                         plan.perm.data_ptr(), sc.data_ptr() if sc is not None else None,
                         plan.tokens, plan.topk, out.data_ptr(), out.stride(0), _stream_ptr(y)),
        "combine",
    )
    return out


def combine_score_grad(grad_out: torch.Tensor, y: torch.Tensor, plan: RoutePlan):
    """d loss / d scores of combine(y, plan, scores): fp32 [tokens, topk],
    grad[t, k] = sum_h grad_out[t, h] * y[perm[t, k], h]."""
    _need_gpu(grad_out, "grad_out")
    for name, t in (("grad_out", grad_out), ("y", y)):
        if t.dtype != torch.bfloat16 or t.dim() != 2:
            raise TypeError(f"{name} must be a 2-D bfloat16 tensor")
    if grad_out.shape[1] != y.shape[1] or grad_out.shape[0] != plan.tokens:
        raise ValueError("grad_out must be [tokens, H] with the H of y")
    g2, y2 = _rows_ok(grad_out), _rows_ok(y)
    out = torch.empty((plan.tokens, plan.topk), dtype=torch.float32, device=y.device)
    lib = _lib.load()
    _lib.check(
        lib.mxgg_combine_score_grad(g2.data_ptr(), g2.stride(0), y2.data_ptr(), y2.shape[0],
                                    y2.shape[1], y2.stride(0), plan.perm.data_ptr(), plan.tokens,
                                    plan.topk, out.data_ptr(), _stream_ptr(y)),
        "combine_score_grad",
    )
    return out
