"""mxfp8gg — MXFP8 grouped GEMM for AMD MI355X (gfx950).

bf16 -> MXFP8 casts, a forward grouped GEMM and a weight-gradient grouped GEMM
over ragged expert groups, the expert FFN's fused SwiGLU casts, and the token
routing (dispatch plan, gather, combine) around them, all as hand-written HIP
kernels in libmxgg.so behind a C ABI (include/mxgg.h).  This package is the
host side: it takes torch tensors, allocates outputs, and calls the library on
the current stream.
"""
from ._lib import MxggError, load as load_library
from .ops import (
    GroupEnds,
    _best_config,
    fused_grouped_fwd,
    fwd_ge,
    grouped_dgrad,
    grouped_mm,
    grouped_mm_swiglu_quant,
    grouped_wgrad,
    offs_to_group_ends,
    padded_token_capacity,
    quant_weight_dual,
    quant_weight_for_dgrad,
    swiglu_backward_quant,
    swiglu_quant,
    to_mxfp8_dim0,
    to_mxfp8_dim1,
    to_mxfp8_dual,
    wgrad_fused,
    wgrad_kernel,
    wgrad_prepare,
    zero_rows_past_groups,
)
from .weight_cache import WeightCastCache
from .autograd import (
    MXFP8ExpertFFN,
    MXFP8GroupedMM,
    MXFP8RoutedExpertFFN,
    moe_ffn,
    moe_ffn_unfused,
    moe_routed_ffn,
    mxfp8_grouped_mm,
)
from .routing import (
    RoutePlan,
    combine,
    combine_score_grad,
    gather_rows,
    gather_to_mxfp8_dual,
    gather_to_mxfp8_dim0,
    route_plan,
)
from .torchao_compat import (
    apply,
    triton_mxfp8_grouped_mm,
    triton_mxfp8_wgrad,
    triton_mxfp8_wgrad_v2,
    triton_to_mxfp8_dim0,
    triton_to_mxfp8_dim1,
)

__all__ = [
    "MxggError", "load_library",
    "to_mxfp8_dim0", "to_mxfp8_dim1", "to_mxfp8_dual", "padded_token_capacity",
    "grouped_mm", "grouped_mm_swiglu_quant", "grouped_wgrad", "grouped_dgrad", "quant_weight_for_dgrad",
    "quant_weight_dual", "swiglu_quant", "swiglu_backward_quant",
    "fused_grouped_fwd", "fwd_ge", "wgrad_fused", "wgrad_prepare", "wgrad_kernel",
    "offs_to_group_ends", "zero_rows_past_groups", "GroupEnds",
    "triton_to_mxfp8_dim0", "triton_to_mxfp8_dim1",
    "triton_mxfp8_grouped_mm", "triton_mxfp8_wgrad", "triton_mxfp8_wgrad_v2", "apply",
    "WeightCastCache",
    "MXFP8GroupedMM", "mxfp8_grouped_mm", "MXFP8ExpertFFN", "moe_ffn", "moe_ffn_unfused",
    "RoutePlan", "route_plan", "gather_rows", "gather_to_mxfp8_dual", "gather_to_mxfp8_dim0",
    "combine",
    "combine_score_grad", "MXFP8RoutedExpertFFN", "moe_routed_ffn",
]
