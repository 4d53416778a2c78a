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

from . import ops, routing


class MXFP8GroupedMM(torch.autograd.Function):
    """y = grouped x . W^T with MXFP8 operands and fp32 accumulation.

    Every operand that the backward pass contracts the other way is cast both
    ways from one read (to_mxfp8_dual / quant_weight_dual): the forward keeps
    the token-axis cast of x and the N-blocked cast of W for backward instead
    of the bf16 tensors, and dY is cast once for dgrad and wgrad together."""

    @staticmethod
    def forward(ctx, x, w, offs, scaling_mode="rceil", weight_cache=None):
        if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
            raise TypeError("x and w must be bfloat16")
        offs = ops._group_ends(offs, w.shape[0], x.device)
        need_dx, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        saved = [offs]
        if need_dw:
            xq, xs, xqt, xst, pad = ops.to_mxfp8_dual(x, offs, scaling_mode)
            saved += [xqt, xst, pad]
        else:
            xq, xs = ops.to_mxfp8_dim0(x, scaling_mode)
        if weight_cache is not None:
            (wq, ws), (wt, wts) = weight_cache.get(w, scaling_mode)
            if need_dx:
                saved += [wt, wts]
        elif need_dx:
            (wq, ws), (wt, wts) = ops.quant_weight_dual(w, scaling_mode)
            saved += [wt, wts]
        else:
            wq, ws = ops.to_mxfp8_dim0(w, scaling_mode)
        y = ops.zero_rows_past_groups(ops.grouped_mm(xq, wq, offs, xs, ws, out_dtype=torch.bfloat16),
                                      offs)
        ctx.save_for_backward(*saved)
        ctx.scaling_mode = scaling_mode
        ctx.w_dtype = w.dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        need_dx, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        saved = list(ctx.saved_tensors)
        offs = saved.pop(0)
        if need_dw:
            xqt, xst, pad = saved[:3]
            saved = saved[3:]
        if need_dx:
            wt, wts = saved[:2]
        mode = ctx.scaling_mode
        dy = dy.to(torch.bfloat16)
        if dy.stride(-1) != 1:
            dy = dy.contiguous()
        dx = dw = None
        if need_dx and need_dw:
            dyq, dys, dyqt, dyst, _ = ops.to_mxfp8_dual(dy, offs, mode)
        elif need_dx:
            dyq, dys = ops.to_mxfp8_dim0(dy, mode)
        elif need_dw:
            dyqt, dyst, _ = ops.to_mxfp8_dim1(dy, offs, mode)
        if need_dx:
            dx = ops.zero_rows_past_groups(
                ops.grouped_mm(dyq, wt, offs, dys, wts, out_dtype=torch.bfloat16), offs)
        if need_dw:
            dw = ops.grouped_wgrad(dyqt, xqt, pad, dyst, xst, out_dtype=ctx.w_dtype)
        return dx, dw, None, None, None


def mxfp8_grouped_mm(x: torch.Tensor, w: torch.Tensor, offs: torch.Tensor,
                     scaling_mode: str = "rceil", weight_cache=None) -> torch.Tensor:
    """Differentiable MXFP8 grouped GEMM: x bf16 [M, K], w bf16 [E, N, K],
    offs int32 group ends [E] (or [E+1] with a leading 0) -> bf16 [M, N].
    Rows after the last group end get zeros, in the output and in x's
    gradient (the raw op grouped_mm leaves them untouched).  weight_cache: an
    optional WeightCastCache reusing w's casts while w is unchanged."""
    return MXFP8GroupedMM.apply(x, w, offs, scaling_mode, weight_cache)


class MXFP8ExpertFFN(torch.autograd.Function):
    """y = (SiLU(x . Wg^T) * (x . Wu^T)) . Wd^T per expert group, every GEMM in
    MXFP8, the activation fused with the casts around it.

    forward : x and both weights cast both ways from one read each (the
              token-axis / N-blocked casts are kept for backward) -> gate+up
              GEMM writing h = [gate | up] (bf16, kept) and the cast of
              SwiGLU(h) from its epilogue -> down GEMM
    backward: dY cast both ways; dA = dY . Wd (MXFP8 dgrad); one kernel turns
              (h, dA) into the row-wise and token-axis casts of dh =
              [d_gate | d_up] and the token-axis cast of a; then dWd = dY^T . a,
              dX = dh . Wgu and dWgu = dh^T . X, all MXFP8.
    """

    @staticmethod
    def forward(ctx, x, w_gate_up, w_down, offs, scaling_mode="rceil", weight_cache=None):
        E, ends = _check_ffn(x, w_gate_up, w_down, offs)
        wcast = weight_cache.get if weight_cache is not None else ops.quant_weight_dual
        xq, xs, xqt, xst, _ = ops.to_mxfp8_dual(x, ends, scaling_mode)
        (wq, ws), (wgt, wgts) = wcast(w_gate_up, scaling_mode)
        aq, as_, h = _gate_up_act(xq, xs, wq, ws, ends, scaling_mode, keep_h=True)
        (dq, ds), (wdt, wdts) = wcast(w_down, scaling_mode)
        y = ops.zero_rows_past_groups(ops.grouped_mm(aq, dq, ends, as_, ds, out_dtype=torch.bfloat16),
                                      ends)
        ctx.save_for_backward(ends, h, xqt, xst, wgt, wgts, wdt, wdts)
        ctx.scaling_mode = scaling_mode
        ctx.dtypes = (w_gate_up.dtype, w_down.dtype)
        return y

    @staticmethod
    def backward(ctx, dy):
        ends, h, xqt, xst, wgt, wgts, wdt, wdts = ctx.saved_tensors
        mode = ctx.scaling_mode
        dy = dy.to(torch.bfloat16)
        if dy.stride(-1) != 1:
            dy = dy.contiguous()
        dyq, dys, dyqt, dyst, _ = ops.to_mxfp8_dual(dy, ends, mode)
        da = ops.grouped_mm(dyq, wdt, ends, dys, wdts, out_dtype=torch.bfloat16)
        act = ops.swiglu_backward_quant(h, da, ends, mode)
        pad = act["offs_pad"]
        dx = dwgu = dwd = None
        if ctx.needs_input_grad[2]:
            dwd = ops.grouped_wgrad(dyqt, act["a_qt"], pad, dyst, act["a_st"], out_dtype=ctx.dtypes[1])
        if ctx.needs_input_grad[0]:
            dx = ops.zero_rows_past_groups(
                ops.grouped_mm(act["dh_q"], wgt, ends, act["dh_s"], wgts, out_dtype=torch.bfloat16),
                ends)
        if ctx.needs_input_grad[1]:
            dwgu = ops.grouped_wgrad(act["dh_qt"], xqt, pad, act["dh_st"], xst,
                                     out_dtype=ctx.dtypes[0])
        return dx, dwgu, dwd, None, None, None


def _check_ffn(x, w_gate_up, w_down, offs):
    for name, t in (("x", x), ("w_gate_up", w_gate_up), ("w_down", w_down)):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16")
    E, F2, H = w_gate_up.shape
    if tuple(w_down.shape) != (E, H, F2 // 2) or x.shape[-1] != H:
        raise ValueError("shapes must be x [M, H], w_gate_up [E, 2F, H], w_down [E, H, F]")
    return E, (ops._group_ends(offs, E, x.device) if offs is not None else None)


def _weight_dim0(w, scaling_mode, weight_cache):
    if weight_cache is not None:
        return weight_cache.get(w, scaling_mode)[0]
    return ops.to_mxfp8_dim0(w, scaling_mode)


def _gate_up_act(xq, xs, wq, ws, ends, scaling_mode, keep_h=False):
    """MXFP8 cast of SiLU(gate) * up of the gate+up projection (and, with
    keep_h, the bf16 projection h itself as a third result): one fused kernel
    when the intermediate size allows (F % 128 == 0, activations under 2 GiB),
    else the GEMM's bf16 output through the standalone SwiGLU cast.  On the
    rows inside the groups the fused kernel gives the bits of the unsplit GEMM
    followed by that cast; the training and forward-only passes of one shape
    take the same branch."""
    F2 = wq.shape[1]
    if F2 % 256 == 0 and (xq.shape[0] == 0 or
                          (xq.shape[0] - 1) * xq.stride(0) + xq.shape[1] <= ops._MAX_OPERAND_BYTES):
        return ops.grouped_mm_swiglu_quant(xq, wq, ends, xs, ws, scaling_mode, return_h=keep_h)
    h = ops.grouped_mm(xq, wq, ends, xs, ws, out_dtype=torch.bfloat16)
    aq, as_ = ops.swiglu_quant(h, scaling_mode)
    return (aq, as_, h) if keep_h else (aq, as_)


def _ffn_forward_only(x, w_gate_up, w_down, offs, scaling_mode, weight_cache=None):
    _, ends = _check_ffn(x, w_gate_up, w_down, offs)
    xq, xs = ops.to_mxfp8_dim0(x, scaling_mode)
    wq, ws = _weight_dim0(w_gate_up, scaling_mode, weight_cache)
    aq, as_ = _gate_up_act(xq, xs, wq, ws, ends, scaling_mode)
    dq, ds = _weight_dim0(w_down, scaling_mode, weight_cache)
    y = ops.grouped_mm(aq, dq, ends, as_, ds, out_dtype=torch.bfloat16)
    return ops.zero_rows_past_groups(y, ends) if ends is not None else y


def moe_ffn(x: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor,
            offs: torch.Tensor, scaling_mode: str = "rceil", weight_cache=None) -> torch.Tensor:
    """One DeepSeek-V3-style expert FFN over routed tokens (the layer step of
    the reference's e2e_bench.py:56-134): gate+up projection with the fused
    weight w_gate_up [E, 2F, H] (gate rows first), SiLU(gate) * up, down
    projection w_down [E, H, F].  x: bf16 [M, H], tokens grouped by expert with
    cumulative ends `offs`.  Rows after the last group end get zero output and
    zero input gradient.  weight_cache: an optional WeightCastCache reusing the
    weights' casts while they are unchanged (micro-batches between optimizer
    steps, evaluation)."""
    if not torch.is_grad_enabled() or not any(
            t.requires_grad for t in (x, w_gate_up, w_down)):
        return _ffn_forward_only(x, w_gate_up, w_down, offs, scaling_mode, weight_cache)
    return MXFP8ExpertFFN.apply(x, w_gate_up, w_down, offs, scaling_mode, weight_cache)


def moe_ffn_unfused(x: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor,
                    offs: torch.Tensor, scaling_mode: str = "rceil") -> torch.Tensor:
    """The same layer composed from two MXFP8GroupedMM calls and torch's eager
    bf16 SiLU * up (the reference's own composition, e2e_bench.py:56-61); kept
    as the comparison point for the fused path."""
    h = mxfp8_grouped_mm(x, w_gate_up, offs, scaling_mode)
    f = w_down.shape[2]
    a = torch.nn.functional.silu(h[:, :f]) * h[:, f:]
    return mxfp8_grouped_mm(a, w_down, offs, scaling_mode)


class MXFP8RoutedExpertFFN(torch.autograd.Function):
    """out = combine(FFN(gather(x)), scores): the expert FFN of MXFP8ExpertFFN
    between the top-k dispatch and combine of a MoE layer on one GPU.

    forward : route plan (device) -> both casts of the routed x read straight
              from token order -> gate+up GEMM writing h (bf16, kept) and the
              cast of SwiGLU(h) from its epilogue -> down GEMM -> combine
              (score-weighted, fp32 sum over k)
    backward: the routed dY = bf16(dOut[t] * score[s]) is never written: its two
              casts are gathered from dOut; then as MXFP8ExpertFFN; the routed
              dX is summed back over k; d scores = dOut . routed output.
    """

    @staticmethod
    def forward(ctx, x, expert_idx, scores, w_gate_up, w_down, pad_multiple=32,
                scaling_mode="rceil", weight_cache=None):
        E, _ = _check_ffn(x, w_gate_up, w_down, None)
        plan = routing.route_plan(expert_idx, E, pad_multiple)
        wcast = weight_cache.get if weight_cache is not None else ops.quant_weight_dual
        xq, xs, xqt, xst, _ = routing.gather_to_mxfp8_dual(x, plan, scaling_mode)
        (wq, ws), (wgt, wgts) = wcast(w_gate_up, scaling_mode)
        aq, as_, h = _gate_up_act(xq, xs, wq, ws, plan.offs, scaling_mode, keep_h=True)
        (dq, ds), (wdt, wdts) = wcast(w_down, scaling_mode)
        y = ops.grouped_mm(aq, dq, plan.offs, as_, ds, out_dtype=torch.bfloat16)
        sc = scores.to(torch.float32).contiguous() if scores is not None else None
        out = routing.combine(y, plan, sc)
        ctx.save_for_backward(plan.perm, plan.src, plan.offs, plan.counts, h, xqt, xst, wgt, wgts,
                              wdt, wdts, y, sc if sc is not None else torch.empty(0))
        ctx.plan_meta = (plan.tokens, plan.topk, plan.num_experts, plan.pad_multiple)
        ctx.has_scores = sc is not None
        ctx.scaling_mode = scaling_mode
        ctx.dtypes = (x.dtype, w_gate_up.dtype, w_down.dtype,
                      scores.dtype if scores is not None else None)
        return out

    @staticmethod
    def backward(ctx, dout):
        perm, src, offs, counts, h, xqt, xst, wgt, wgts, wdt, wdts, y, sc = ctx.saved_tensors
        plan = routing.RoutePlan(perm, src, offs, counts, *ctx.plan_meta)
        mode = ctx.scaling_mode
        sc = sc if ctx.has_scores else None
        dout = dout.to(torch.bfloat16)
        if dout.stride(-1) != 1:
            dout = dout.contiguous()
        dx = dsc = dwgu = dwd = None
        if ctx.has_scores and ctx.needs_input_grad[2]:
            dsc = routing.combine_score_grad(dout, y, plan).to(ctx.dtypes[3])
        dyq, dys, dyqt, dyst, _ = routing.gather_to_mxfp8_dual(dout, plan, mode, row_scale=sc)
        da = ops.grouped_mm(dyq, wdt, offs, dys, wdts, out_dtype=torch.bfloat16)
        act = ops.swiglu_backward_quant(h, da, offs, mode)
        pad = act["offs_pad"]
        if ctx.needs_input_grad[4]:
            dwd = ops.grouped_wgrad(dyqt, act["a_qt"], pad, dyst, act["a_st"],
                                    out_dtype=ctx.dtypes[2])
        if ctx.needs_input_grad[0]:
            dxr = ops.grouped_mm(act["dh_q"], wgt, offs, act["dh_s"], wgts,
                                 out_dtype=torch.bfloat16)
            dx = routing.combine(dxr, plan, None)
        if ctx.needs_input_grad[3]:
            dwgu = ops.grouped_wgrad(act["dh_qt"], xqt, pad, act["dh_st"], xst,
                                     out_dtype=ctx.dtypes[1])
        return dx, None, dsc, dwgu, dwd, None, None, None


def _routed_forward_only(x, expert_idx, scores, w_gate_up, w_down, pad_multiple, scaling_mode,
                         weight_cache=None):
    E, _ = _check_ffn(x, w_gate_up, w_down, None)
    plan = routing.route_plan(expert_idx, E, pad_multiple)
    xq, xs = routing.gather_to_mxfp8_dim0(x, plan, scaling_mode)
    wq, ws = _weight_dim0(w_gate_up, scaling_mode, weight_cache)
    aq, as_ = _gate_up_act(xq, xs, wq, ws, plan.offs, scaling_mode)
    dq, ds = _weight_dim0(w_down, scaling_mode, weight_cache)
    y = ops.grouped_mm(aq, dq, plan.offs, as_, ds, out_dtype=torch.bfloat16)
    return routing.combine(y, plan, scores)


def moe_routed_ffn(x: torch.Tensor, expert_idx: torch.Tensor, scores: torch.Tensor | None,
                   w_gate_up: torch.Tensor, w_down: torch.Tensor, pad_multiple: int = 32,
                   scaling_mode: str = "rceil", weight_cache=None) -> torch.Tensor:
    """The routed experts of one MoE layer on one GPU: every token t goes to the
    experts expert_idx[t, :] (int [T, topk]; ids outside [0, E) are dropped),
    through moe_ffn's MXFP8 expert FFN, and comes back as
    sum_k scores[t, k] * expert_output (scores [T, topk] or None for a plain
    sum).  x: bf16 [T, H]; w_gate_up [E, 2F, H]; w_down [E, H, F].  Each
    expert's rows are padded to pad_multiple (the reference's dispatcher uses
    32, port_mxfp8.py:214).  Differentiable in x, scores and both weights;
    without autograd (no_grad, or nothing requiring grad) only the row-wise
    casts are made and nothing is kept for backward."""
    if not torch.is_grad_enabled() or not any(
            t is not None and t.requires_grad for t in (x, scores, w_gate_up, w_down)):
        return _routed_forward_only(x, expert_idx, scores, w_gate_up, w_down, pad_multiple,
                                    scaling_mode, weight_cache)
    return MXFP8RoutedExpertFFN.apply(x, expert_idx, scores, w_gate_up, w_down, pad_multiple,
                                      scaling_mode, weight_cache)
