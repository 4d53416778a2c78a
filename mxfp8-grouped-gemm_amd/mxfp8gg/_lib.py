"""ctypes binding of libmxgg.so (the C ABI declared in include/mxgg.h).

The library is loaded lazily on first use.  There is no fallback: if the
shared library is missing, or no ROCm GPU is visible, every compute entry point
raises instead of silently computing on the CPU.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmxgg.so"

# mxgg_status
OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_SHAPE = 2
ERR_ALIGNMENT = 3
ERR_UNSUPPORTED = 4
ERR_DEVICE = 5
ERR_LAUNCH = 6

SCALE_RCEIL = 0
SCALE_FLOOR = 1
CVT_SOFTWARE = 0x100  # verification-only: bit-level e4m3 encoder instead of v_cvt_pk_fp8_f32

OUT_BF16 = 0
OUT_F32 = 1

SCALES_ROW_MAJOR = 0
SCALES_BLOCK_MAJOR = 1

OFFS_ENDS = 0
OFFS_SIZES = 1
OFFS_AUTO = 2

ABI_VERSION = 13

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int

# name -> (restype, argtypes); must list every function of include/mxgg.h
SIGNATURES = {
    "mxgg_abi_version": (_I, []),
    "mxgg_status_string": (ctypes.c_char_p, [_I]),
    "mxgg_last_error": (ctypes.c_char_p, []),
    "mxgg_quant_dim0": (_I, [_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _I, _I, _P]),
    "mxgg_quant_dim1": (
        _I,
        [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _I, _P, _I, _P],
    ),
    "mxgg_quant_dual": (
        _I,
        [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I, _P, _I,
         _P],
    ),
    "mxgg_swiglu_quant_dim0": (
        _I, [_P, _P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _I, _I, _P],
    ),
    "mxgg_swiglu_bwd_quant": (
        _I,
        [_P, _P, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _P, _I64,
         _P, _I64, _P, _I64, _P, _I64, _P, _P, _I64, _I, _I, _P],
    ),
    "mxgg_scales_to_block_major": (
        _I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P],
    ),
    "mxgg_offs_to_group_ends": (_I, [_P, _I64, _I64, _I, _P, _P]),
    "mxgg_zero_rows_past_groups": (_I, [_P, _I64, _I64, _I64, _P, _I64, _P]),
    "mxgg_grouped_fwd": (
        _I,
        [_P, _I64, _P, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64,
         _P, _I64, _I, _P],
    ),
    "mxgg_grouped_fwd_workspace_bytes": (_I64, []),
    "mxgg_grouped_fwd_swiglu_quant": (
        _I,
        [_P, _I64, _P, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64,
         _P, _I64, _P, _I64, _I, _I, _P],
    ),
    "mxgg_grouped_fwd_swiglu_quant_keep_h": (
        _I,
        [_P, _I64, _P, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64,
         _P, _I64, _P, _I64, _P, _I64, _I, _I, _P],
    ),
    "mxgg_grouped_fwd_split": (
        _I,
        [_P, _I64, _P, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64,
         _P, _I64, _I, _P, _I64, _P],
    ),
    "mxgg_grouped_fwd_split_noalloc": (
        _I,
        [_P, _I64, _P, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64,
         _P, _I64, _I, _P],
    ),
    "mxgg_grouped_wgrad": (
        _I,
        [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I, _I64, _P],
    ),
    "mxgg_grouped_wgrad_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64]),
    "mxgg_grouped_wgrad_split": (
        _I,
        [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I, _I64, _P,
         _I64, _P],
    ),
    "mxgg_grouped_wgrad_strided": (
        _I,
        [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _I64, _I,
         _I64, _P, _I64, _P],
    ),
    "mxgg_route_plan": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P]),
    "mxgg_route_plan_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "mxgg_route_plan_ws": (
        _I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _I64, _P]),
    "mxgg_gather_rows": (_I, [_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _P]),
    "mxgg_gather_quant_dual": (
        _I,
        [_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _P, _I64,
         _P, _I64, _I, _P, _I, _P],
    ),
    "mxgg_gather_quant_dim0": (
        _I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _I, _I, _P],
    ),
    "mxgg_combine": (_I, [_P, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _I64, _P]),
    "mxgg_combine_score_grad": (
        _I, [_P, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, _P, _P],
    ),
}


class MxggError(RuntimeError):
    """A libmxgg entry point returned a non-OK status."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load libmxgg.so and attach argument types (idempotent)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it first (python __graft_entry__.py build, or "
                "mxfp8gg._build.build()); there is no CPU fallback"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        v = lib.mxgg_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"libmxgg ABI version {v}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(status: int, what: str) -> None:
    if status == OK:
        return
    lib = load()
    detail = lib.mxgg_last_error().decode(errors="replace")
    name = lib.mxgg_status_string(status).decode(errors="replace")
    msg = f"{what}: {name}: {detail}"
    if status in (ERR_INVALID_ARGUMENT, ERR_SHAPE, ERR_ALIGNMENT, ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise MxggError(status, msg)
