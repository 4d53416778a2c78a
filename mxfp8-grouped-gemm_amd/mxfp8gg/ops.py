"""Host side of the MXFP8 grouped-GEMM path: torch tensors in, libmxgg out.

PyTorch only provides device memory and the current stream; every byte of
arithmetic runs in the HIP kernels of libmxgg.so.  Outputs are allocated from
torch's caching allocator and handed to the C ABI as raw pointers.  Nothing
here synchronises with the host: group offsets stay on the device.

Reference entry points mirrored here (all paths under the reference repo):
  fused_grouped_fwd   fused_fwd.py:172-229
  fwd_ge              fwd_final.py:121-131
  wgrad_fused         wgrad_fused.py:34-71
  wgrad_prepare       wgrad_fused.py:74-103
  wgrad_kernel        wgrad_fused.py:106-112
  _best_config        wgrad_fused.py:22-31
"""
from __future__ import annotations

import torch

from . import _lib

_FP8 = torch.float8_e4m3fn
_E8M0 = getattr(torch, "float8_e8m0fnu", None)

_MODES = {"rceil": _lib.SCALE_RCEIL, "floor": _lib.SCALE_FLOOR}


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def _stream_ptr(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _need_gpu(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(
            f"{name} is on {t.device}; the MXFP8 kernels run on a ROCm GPU only "
            "(there is no CPU implementation)"
        )


def _mode(scaling_mode) -> int:
    if isinstance(scaling_mode, int):
        return scaling_mode
    key = str(getattr(scaling_mode, "value", scaling_mode)).lower()
    if key not in _MODES:
        raise ValueError(f"scaling_mode must be one of {sorted(_MODES)}, got {scaling_mode!r}")
    return _MODES[key]


def _as_u8(t: torch.Tensor | None, name: str) -> torch.Tensor | None:
    """Scale / payload tensors as raw bytes (uint8 view, no copy)."""
    if t is None:
        return None
    if t.dtype == torch.uint8:
        return t
    if t.dtype == _FP8 or (_E8M0 is not None and t.dtype == _E8M0) or t.dtype == torch.int8:
        return t.view(torch.uint8)
    raise TypeError(f"{name}: expected uint8 / float8_e8m0fnu / float8_e4m3fn, got {t.dtype}")


def _rowmajor(t: torch.Tensor) -> torch.Tensor:
    """Last dimension contiguous (copy only if it is not)."""
    return t if t.stride(-1) == 1 else t.contiguous()


def _group_ends(offs: torch.Tensor, num_groups: int, device) -> torch.Tensor:
    """Accept [E] cumulative ends (torch._grouped_mm convention, used by every
    caller of the reference) or [E+1] with a leading 0 (the form documented
    at fused_fwd.py:7,181); return int32 [E] on the device."""
    if not isinstance(offs, torch.Tensor):
        offs = torch.as_tensor(offs, dtype=torch.int32)
    if offs.dim() != 1:
        raise ValueError(f"offs must be 1-D, got shape {tuple(offs.shape)}")
    if offs.numel() == num_groups + 1:
        offs = offs[1:]
    elif offs.numel() != num_groups:
        raise ValueError(
            f"offs has {offs.numel()} entries; expected {num_groups} group ends "
            f"(or {num_groups + 1} with a leading 0)"
        )
    if offs.device != device:
        offs = offs.to(device, non_blocking=True)
    if offs.dtype != torch.int32:
        offs = offs.to(torch.int32)
    return offs.contiguous()


class GroupEnds(torch.Tensor):
    """int32 cumulative group ends that this library wrote: the padded ends of
    its token-axis casts and of SwiGLU backward, routing plans, and
    offs_to_group_ends.  The reference-named wgrad entry points always read a
    GroupEnds as ends, never as group sizes (a degenerate routing, every token
    in the first expert, can make padded ends look like sizes).

    The type is part of the tensor, so it survives what copies the values
    unchanged: clone, copy.deepcopy, detach, to / cpu / cuda / int / long,
    contiguous, pin_memory, and torch.cat / torch.stack of GroupEnds only.  Anything
    else (arithmetic, indexing, diff) returns a plain tensor: the library no
    longer knows what its values mean."""

    _KEEP = frozenset({
        torch.Tensor.clone, torch.clone, torch.Tensor.detach, torch.detach,
        torch.Tensor.to, torch.Tensor.cpu, torch.Tensor.cuda, torch.Tensor.int,
        torch.Tensor.long, torch.Tensor.contiguous, torch.Tensor.pin_memory,
        torch.Tensor.share_memory_,
    })
    _JOIN = frozenset({torch.cat, torch.concat, torch.stack})

    def __deepcopy__(self, memo):
        out = self.as_subclass(torch.Tensor).clone().as_subclass(GroupEnds)
        memo[id(self)] = out
        return out

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        with torch._C.DisableTorchFunctionSubclass():
            out = func(*args, **kwargs)
        if not isinstance(out, torch.Tensor):
            return out
        if func in cls._KEEP:
            return out.as_subclass(cls)
        if func in cls._JOIN:
            parts = args[0] if args else kwargs.get("tensors", ())
            if parts and all(isinstance(t, cls) for t in parts):
                return out.as_subclass(cls)
        return out


def _mark_ends(t):
    """Mark a tensor this library wrote as cumulative group ends (GroupEnds)."""
    if t is None or isinstance(t, GroupEnds):
        return t
    return t.as_subclass(GroupEnds)


def _warn_if_ambiguous(offs: torch.Tensor, tokens: int) -> None:
    """With MXGG_CHECK_OFFS=1: warn when an "auto" offs vector fits both
    readings (non-decreasing, so valid as ends, and adding up to exactly
    `tokens` with its last entry below it, so valid as sizes).  Off by default:
    the check reads offs back to the host, which the library otherwise never
    does."""
    import os
    import warnings

    if os.environ.get("MXGG_CHECK_OFFS", "0") in ("", "0"):
        return
    v = offs.detach().to("cpu", torch.int64)
    if v.numel() > 1 and bool((v[1:] >= v[:-1]).all()) and int(v.sum()) == tokens \
            and int(v[-1]) < tokens:
        warnings.warn(f"offs {v.tolist()} reads as group sizes and as cumulative ends for "
                      f"{tokens} tokens; the auto rule takes sizes, pass offs_kind= to choose",
                      RuntimeWarning, stacklevel=3)


_OFFS_KINDS = {"ends": _lib.OFFS_ENDS, "sizes": _lib.OFFS_SIZES, "auto": _lib.OFFS_AUTO}


def offs_to_group_ends(offs: torch.Tensor, tokens: int, offs_kind: str = "auto") -> torch.Tensor:
    """Cumulative group ends (int32 [E], on the device) from an `offs` vector
    given as cumulative ends ("ends"), per-group sizes ("sizes"), or either
    ("auto": sizes when they add up to exactly `tokens` and the last entry is
    below `tokens`, ends otherwise), decided on the device by one small kernel
    (mxgg_offs_to_group_ends), with no host sync.  Tensors this library
    returned as group ends (the padded ends of its token-axis casts, routing
    plans: GroupEnds, also after clone() / to() / cpu()) are always read as
    ends.  Set MXGG_CHECK_OFFS=1 to be warned when an "auto" vector fits both
    readings (costs a device-to-host read)."""
    if offs_kind not in _OFFS_KINDS:
        raise ValueError(f"offs_kind must be one of {sorted(_OFFS_KINDS)}, got {offs_kind!r}")
    if isinstance(offs, GroupEnds):
        offs_kind = "ends"
    if not isinstance(offs, torch.Tensor) or offs.dim() != 1:
        raise ValueError("offs must be a 1-D tensor")
    _need_gpu(offs, "offs")
    if offs_kind == "auto":
        _warn_if_ambiguous(offs, tokens)
    src = offs.to(torch.int32).contiguous()
    out = torch.empty_like(src)
    _lib.check(_lib.load().mxgg_offs_to_group_ends(src.data_ptr(), src.numel(), int(tokens),
                                                   _OFFS_KINDS[offs_kind], out.data_ptr(),
                                                   _stream_ptr(src)), "offs_to_group_ends")
    return _mark_ends(out)


def zero_rows_past_groups(out: torch.Tensor, offs: torch.Tensor) -> torch.Tensor:
    """Set the rows of a row-major 2-D `out` past the last group end to zero
    (the rows no grouped GEMM writes), reading the ends on the device."""
    _need_gpu(out, "out")
    if out.dim() != 2 or out.stride(-1) != 1:
        raise ValueError("out must be a row-major 2-D tensor")
    E = offs.numel()
    ends = _group_ends(offs, E, out.device)
    esz = out.element_size()
    _lib.check(_lib.load().mxgg_zero_rows_past_groups(
        out.data_ptr(), out.shape[0], out.shape[1] * esz, out.stride(0) * esz, ends.data_ptr(),
        E, _stream_ptr(out)), "zero_rows_past_groups")
    return out


def _ld16(n: int) -> int:
    return max(16, (n + 15) // 16 * 16)


def _block_major_buffer(rows: int, nblk: int, device) -> torch.Tensor:
    """Storage for E8M0 scales laid out block-major: [nblk][round_up(rows, 16)]."""
    return torch.empty((nblk, _ld16(rows)), dtype=torch.uint8, device=device)


def _readable(t: torch.Tensor) -> int:
    """Bytes of storage from t's first element to the end of its storage."""
    return t.untyped_storage().nbytes() - t.storage_offset() * t.element_size()


def _scales_2d(s: torch.Tensor, rows: int, nblk: int, name: str):
    """Logical [rows, nblk] E8M0 scales -> (tensor, block-major stride) for the
    GEMM kernels.  A block-major view (stride (1, ld), e.g. what this library's
    casts return) is used in place; anything else is re-laid on the device."""
    s = _as_u8(s, name)
    _need_gpu(s, name)
    if tuple(s.shape) != (rows, nblk):
        raise ValueError(f"{name} shape {tuple(s.shape)} != {(rows, nblk)}")
    if (s.stride(0) == 1 or rows == 1) and s.stride(1) >= rows and s.stride(1) % 4 == 0 \
            and s.data_ptr() % 4 == 0 and nblk > 0 \
            and _readable(s) >= (nblk - 1) * s.stride(1) + (rows + 3) // 4 * 4:
        return s, s.stride(1)
    src = s.contiguous()
    dst = _block_major_buffer(rows, nblk, s.device)
    lib = _lib.load()
    _lib.check(lib.mxgg_scales_to_block_major(src.data_ptr(), 1, rows, nblk, 0, nblk,
                                              dst.data_ptr(), 0, dst.stride(0),
                                              _stream_ptr(s)), "scales_to_block_major")
    return dst, dst.stride(0)


def _scales_3d(s: torch.Tensor, E: int, rows: int, nblk: int, name: str):
    """Logical [E, rows, nblk] scales -> (tensor, expert stride, block stride),
    block-major within each expert (the expert stride may interleave experts
    inside a block-row, as the cast of a flattened [E*rows, K] tensor does)."""
    s = _as_u8(s, name)
    _need_gpu(s, name)
    if tuple(s.shape) != (E, rows, nblk):
        raise ValueError(f"{name} shape {tuple(s.shape)} != {(E, rows, nblk)}")
    st = s.stride()
    if (st[1] == 1 or rows == 1) and st[2] % 4 == 0 and (E == 1 or st[0] % 4 == 0) \
            and s.data_ptr() % 4 == 0 and st[2] >= rows and (E == 1 or st[0] >= rows) \
            and _readable(s) >= (E - 1) * st[0] + (nblk - 1) * st[2] + (rows + 3) // 4 * 4:
        return s, st[0], st[2]
    src = s.contiguous()
    ld = _ld16(rows)
    dst = torch.empty((E, nblk, ld), dtype=torch.uint8, device=s.device)
    lib = _lib.load()
    _lib.check(lib.mxgg_scales_to_block_major(src.data_ptr(), E, rows, nblk, rows * nblk, nblk,
                                              dst.data_ptr(), nblk * ld, ld, _stream_ptr(s)),
               "scales_to_block_major")
    return dst, nblk * ld, ld


def _out_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return _lib.OUT_BF16
    if dtype == torch.float32:
        return _lib.OUT_F32
    raise ValueError(f"out_dtype must be torch.bfloat16 or torch.float32, got {dtype}")


# ---------------------------------------------------------------------------
# bf16 -> MXFP8 casts
# ---------------------------------------------------------------------------
def _layout_code(scale_layout: str) -> int:
    if scale_layout == "block":
        return _lib.SCALES_BLOCK_MAJOR
    if scale_layout == "row":
        return _lib.SCALES_ROW_MAJOR
    raise ValueError(f"scale_layout must be 'block' or 'row', got {scale_layout!r}")


def to_mxfp8_dim0(x: torch.Tensor, scaling_mode="rceil", scale_layout: str = "block"):
    """Row-wise MXFP8: 1x32 blocks along the last dimension.

    x: bf16 [..., K] (K % 32 == 0).  Returns (q float8_e4m3fn [..., K],
    scales uint8 [..., K/32]) with E8M0 bytes (2^(b-127)).  scale_layout
    "block" (default): the scales are a view of block-major storage
    ([K/32][rows], what the GEMM kernels read, so they take it without a
    conversion); "row": contiguous row-major scales, written so by the cast
    itself (what torchao's casts return; a GEMM call converts them).
    """
    _need_gpu(x, "x")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"x must be bfloat16, got {x.dtype}")
    shape = x.shape
    K = shape[-1]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
    rows = x2.shape[0]
    nblk = K // 32
    layout = _layout_code(scale_layout)
    q = torch.empty((rows, K), dtype=_FP8, device=x.device)
    if layout == _lib.SCALES_ROW_MAJOR:
        buf = torch.empty((rows, nblk), dtype=torch.uint8, device=x.device)
    else:
        buf = _block_major_buffer(rows, nblk, x.device)
    lib = _lib.load()
    _lib.check(
        lib.mxgg_quant_dim0(x2.data_ptr(), rows, K, x2.stride(0), q.data_ptr(), q.stride(0),
                            buf.data_ptr(), max(buf.stride(0), 1), layout,
                            _mode(scaling_mode), _stream_ptr(x)),
        "quant_dim0",
    )
    if layout == _lib.SCALES_ROW_MAJOR:
        return q.reshape(shape), buf.reshape(tuple(shape[:-1]) + (nblk,))
    lead = tuple(shape[:-1])
    lead_strides = []
    acc = 1
    for d in reversed(lead):
        lead_strides.append(acc)
        acc *= d
    s = buf.as_strided(lead + (nblk,), tuple(reversed(lead_strides)) + (buf.stride(0),))
    return q.reshape(shape), s


def padded_token_capacity(num_tokens: int, num_groups: int | None) -> int:
    """Columns of the dim1 output.

    Ungrouped: the tokens rounded up to 32.  Grouped: room for every group
    padded to 32 tokens, rounded up to 128 so that each row starts on a
    128-byte cache line (the wgrad GEMM streams whole lines)."""
    if not num_groups:
        return (num_tokens + 31) // 32 * 32
    return (num_tokens + 31 * num_groups + 127) // 128 * 128


def to_mxfp8_dim1(x: torch.Tensor, offs: torch.Tensor | None = None, scaling_mode="rceil",
                  scale_layout: str = "block"):
    """Token-axis MXFP8 for the wgrad operands, written transposed.

    x: bf16 [M, C] (tokens x features).  Blocks of 32 run along M and restart
    at each group boundary of `offs` (cumulative ends, int32, on the device);
    each group is zero-padded to a multiple of 32 tokens.
    Returns (qt float8_e4m3fn [C, M_pad], st uint8 [C, M_pad/32], offs_pad)
    where offs_pad are the padded cumulative ends (int32 [E], None without
    offs) and M_pad = padded_token_capacity(M, E) >= offs_pad[-1].  st is a
    view of block-major storage ([M_pad/32][C]) with scale_layout "block"
    (default), contiguous row-major with "row".
    """
    _need_gpu(x, "x")
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise TypeError("x must be a 2-D bfloat16 tensor")
    M, C = x.shape
    x2 = x if (x.stride(-1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0) else x.contiguous()
    E = None
    ends = None
    ends_pad = None
    if offs is not None:
        E = offs.numel()
        ends = _group_ends(offs, E, x.device)
        ends_pad = torch.empty(E, dtype=torch.int32, device=x.device)
    cap = padded_token_capacity(M, E)
    layout = _layout_code(scale_layout)
    qt = torch.empty((C, cap), dtype=_FP8, device=x.device)
    if layout == _lib.SCALES_ROW_MAJOR:
        buf = torch.empty((C, cap // 32), dtype=torch.uint8, device=x.device)
    else:
        buf = _block_major_buffer(C, cap // 32, x.device)
    lib = _lib.load()
    _lib.check(
        lib.mxgg_quant_dim1(
            x2.data_ptr(), M, C, x2.stride(0),
            ends.data_ptr() if ends is not None else None, E or 0, cap,
            qt.data_ptr(), qt.stride(0), buf.data_ptr(), max(buf.stride(0), 1), layout,
            ends_pad.data_ptr() if ends_pad is not None else None,
            _mode(scaling_mode), _stream_ptr(x),
        ),
        "quant_dim1",
    )
    # logical [C, cap/32]: the buffer itself (row-major) or a view of it
    st = buf if layout == _lib.SCALES_ROW_MAJOR else buf[:, :C].t()
    return qt, st, _mark_ends(ends_pad)


def to_mxfp8_dual(x: torch.Tensor, offs: torch.Tensor | None = None, scaling_mode="rceil"):
    """Both MXFP8 casts of x from one read of it: the row-wise cast of
    to_mxfp8_dim0 and the token-axis cast of to_mxfp8_dim1, for operands a
    training step contracts both ways (X and dY of a grouped GEMM).

    x: bf16 [M, C] (C % 32 == 0); offs: token group ends (int32 [E] on the
    device) or None.  Returns (q, s, qt, st, offs_pad) with q, s as
    to_mxfp8_dim0(x) (rows inside the groups) and qt, st, offs_pad as
    to_mxfp8_dim1(x, offs)."""
    _need_gpu(x, "x")
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] % 32 != 0:
        raise TypeError("x must be a 2-D bfloat16 tensor [M, C] with C % 32 == 0")
    M, C = x.shape
    x2 = x if (x.stride(-1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0) else x.contiguous()
    E = ends = ends_pad = None
    if offs is not None:
        E = offs.numel()
        ends = _group_ends(offs, E, x.device)
        ends_pad = torch.empty(E, dtype=torch.int32, device=x.device)
    cap = padded_token_capacity(M, E)
    q = torch.empty((M, C), dtype=_FP8, device=x.device)
    sbuf = _block_major_buffer(M, C // 32, x.device)
    qt = torch.empty((C, cap), dtype=_FP8, device=x.device)
    stbuf = _block_major_buffer(C, cap // 32, x.device)
    lib = _lib.load()
    _lib.check(
        lib.mxgg_quant_dual(
            x2.data_ptr(), M, C, x2.stride(0),
            ends.data_ptr() if ends is not None else None, E or 0, cap,
            q.data_ptr(), C, sbuf.data_ptr(), sbuf.stride(0),
            qt.data_ptr(), cap, stbuf.data_ptr(), stbuf.stride(0), _lib.SCALES_BLOCK_MAJOR,
            ends_pad.data_ptr() if ends_pad is not None else None,
            _mode(scaling_mode), _stream_ptr(x)),
        "quant_dual",
    )
    return q, sbuf[:, :M].t(), qt, stbuf[:, :C].t(), _mark_ends(ends_pad)


def _expert_ends(E: int, N: int, device) -> torch.Tensor:
    return torch.arange(1, E + 1, dtype=torch.int32, device=device) * N


def _weight_t_views(qt: torch.Tensor, st: torch.Tensor, E: int, N: int, K: int):
    """[E, K, N] / [E, K, N/32] views of the token-axis cast of W viewed as
    [E*N, K] with one group per expert (expert e = columns [e*N, (e+1)*N))."""
    wt = qt.as_strided((E, K, N), (N, qt.stride(0), 1))
    # st[k, b] lives at buf[b, k]: strides (1, ld); expert e starts at block-row e*N/32
    wts = st.as_strided((E, K, N // 32), ((N // 32) * st.stride(1), st.stride(0), st.stride(1)))
    return wt, wts


def quant_weight_dual(w: torch.Tensor, scaling_mode="rceil"):
    """Both casts of expert weights W [E, N, K] from one read: returns
    ((wq, ws), (wt, wts)) equal to to_mxfp8_dim0(w) (forward operand, blocks
    along K) and quant_weight_for_dgrad(w) (dgrad operand, blocks along N)."""
    _need_gpu(w, "w")
    if w.dtype != torch.bfloat16 or w.dim() != 3:
        raise TypeError("w must be a 3-D bfloat16 tensor [E, N, K]")
    E, N, K = w.shape
    if N % 32 != 0:
        raise ValueError(f"N={N} must be a multiple of 32 for MXFP8 blocks along N")
    q, s, qt, st, _ = to_mxfp8_dual(w.reshape(E * N, K), _expert_ends(E, N, w.device), scaling_mode)
    return (q.reshape(E, N, K), s.reshape(E, N, K // 32)), _weight_t_views(qt, st, E, N, K)


# ---------------------------------------------------------------------------
# SwiGLU fused with its casts (the expert FFN activation)
# ---------------------------------------------------------------------------
def _gate_up(h: torch.Tensor):
    if h.dtype != torch.bfloat16 or h.dim() != 2 or h.shape[1] % 64 != 0:
        raise TypeError("h must be a 2-D bfloat16 tensor [M, 2F] with F % 32 == 0")
    if h.stride(-1) != 1 or h.stride(0) % 8 != 0 or h.data_ptr() % 16 != 0:
        h = h.contiguous()
    f = h.shape[1] // 2
    return h, h[:, :f], h[:, f:], f


def swiglu_quant(h: torch.Tensor, scaling_mode="rceil", return_bf16: bool = False):
    """a = SiLU(gate) * up of the gate+up projection output h = [gate | up]
    (bf16 [M, 2F]), cast row-wise to MXFP8 in the same pass.

    Returns (q float8_e4m3fn [M, F], scales uint8 [M, F/32]) as to_mxfp8_dim0
    does for a bf16 tensor, plus the bf16 a [M, F] when return_bf16.  a equals
    torch's eager bf16 F.silu(gate) * up (the reference's layer step,
    e2e_bench.py:56-61)."""
    _need_gpu(h, "h")
    h, gate, up, f = _gate_up(h)
    M = h.shape[0]
    q = torch.empty((M, f), dtype=_FP8, device=h.device)
    buf = _block_major_buffer(M, f // 32, h.device)
    a = torch.empty((M, f), dtype=torch.bfloat16, device=h.device) if return_bf16 else None
    lib = _lib.load()
    _lib.check(
        lib.mxgg_swiglu_quant_dim0(
            gate.data_ptr(), up.data_ptr(), h.stride(0), M, f,
            a.data_ptr() if a is not None else None, f,
            q.data_ptr(), f, buf.data_ptr(), buf.stride(0), _lib.SCALES_BLOCK_MAJOR,
            _mode(scaling_mode), _stream_ptr(h)),
        "swiglu_quant_dim0",
    )
    s = buf[:, :M].t()
    return (q, s, a) if return_bf16 else (q, s)


def swiglu_backward_quant(h: torch.Tensor, grad_a: torch.Tensor, offs: torch.Tensor | None,
                          scaling_mode="rceil", return_bf16: bool = False):
    """Backward of a = SiLU(gate) * up fused with the casts of the backward GEMMs.

    h: bf16 [M, 2F] = [gate | up]; grad_a: bf16 [M, F]; offs: token group ends
    (int32 [E] on the device) or None for one group.  Returns a dict:
      dh_q, dh_s      row-wise cast of dh = [d_gate | d_up] [M, 2F]  (dX = dh . W_gate_up)
      dh_qt, dh_st    token-axis cast of dh, [2F, M_pad]            (dW_gate_up)
      a_qt, a_st      token-axis cast of a, [F, M_pad]              (dW_down)
      offs_pad        padded group ends (None without offs)
      dh              bf16 dh [M, 2F] (only with return_bf16)
    Scales are views of block-major storage, as to_mxfp8_dim0 / to_mxfp8_dim1
    return them; M_pad = padded_token_capacity(M, E).  Rows of dh_q past the
    last group end are not written."""
    _need_gpu(h, "h")
    h, gate, up, f = _gate_up(h)
    M = h.shape[0]
    if grad_a.dtype != torch.bfloat16 or tuple(grad_a.shape) != (M, f):
        raise TypeError(f"grad_a must be bfloat16 [{M}, {f}]")
    if grad_a.stride(-1) != 1 or grad_a.stride(0) % 8 != 0 or grad_a.data_ptr() % 16 != 0:
        grad_a = grad_a.contiguous()
    dev = h.device
    E = ends = ends_pad = None
    if offs is not None:
        E = offs.numel()
        ends = _group_ends(offs, E, dev)
        ends_pad = torch.empty(E, dtype=torch.int32, device=dev)
    cap = padded_token_capacity(M, E)
    dh_q = torch.empty((M, 2 * f), dtype=_FP8, device=dev)
    dh_sb = _block_major_buffer(M, 2 * f // 32, dev)
    dh_qt = torch.empty((2 * f, cap), dtype=_FP8, device=dev)
    dh_stb = _block_major_buffer(2 * f, cap // 32, dev)
    a_qt = torch.empty((f, cap), dtype=_FP8, device=dev)
    a_stb = _block_major_buffer(f, cap // 32, dev)
    dh = torch.empty((M, 2 * f), dtype=torch.bfloat16, device=dev) if return_bf16 else None
    lib = _lib.load()
    _lib.check(
        lib.mxgg_swiglu_bwd_quant(
            gate.data_ptr(), up.data_ptr(), h.stride(0), grad_a.data_ptr(), grad_a.stride(0),
            M, f, ends.data_ptr() if ends is not None else None, E or 0, cap,
            dh_q.data_ptr(), 2 * f, dh_sb.data_ptr(), dh_sb.stride(0),
            dh_qt.data_ptr(), cap, dh_stb.data_ptr(), dh_stb.stride(0),
            a_qt.data_ptr(), cap, a_stb.data_ptr(), a_stb.stride(0),
            ends_pad.data_ptr() if ends_pad is not None else None,
            dh.data_ptr() if dh is not None else None, 2 * f,
            _lib.SCALES_BLOCK_MAJOR, _mode(scaling_mode), _stream_ptr(h)),
        "swiglu_bwd_quant",
    )
    out = {
        "dh_q": dh_q, "dh_s": dh_sb[:, :M].t(),
        "dh_qt": dh_qt, "dh_st": dh_stb[:, :2 * f].t(),
        "a_qt": a_qt, "a_st": a_stb[:, :f].t(),
        "offs_pad": _mark_ends(ends_pad),
    }
    if return_bf16:
        out["dh"] = dh
    return out


# ---------------------------------------------------------------------------
# forward grouped GEMM
# ---------------------------------------------------------------------------
_SPLIT_WS_BYTES: dict = {}


def _split_workspace_bytes(device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    n = _SPLIT_WS_BYTES.get(idx)
    if n is None:
        with torch.cuda.device(idx):
            n = int(_lib.load().mxgg_grouped_fwd_workspace_bytes())
        _SPLIT_WS_BYTES[idx] = n
    return n


def _split_workspace(device) -> torch.Tensor:
    """Scratch for mxgg_grouped_fwd_split, from the caching allocator (stream
    ordered, so it can be released as soon as the launch is queued)."""
    return torch.empty(_split_workspace_bytes(device), dtype=torch.uint8, device=device)


def _small_launch(M: int, N: int, E: int, device) -> bool:
    """True when the forward has at most half a round of 256x256 tiles for any
    group sizes: expert g needs ceil((m_g + 3) / 256) m-tiles at most (its
    tiles start up to 3 rows early; the first expert's start at row 0), and
    the sum of those ceilings is at most floor((M + 3(E-1) + 255 E) / 256)."""
    units = (_split_workspace_bytes(device) - 16384) // (256 * 256 * 4)
    m_tiles = (M + 3 * (E - 1) + 255 * E) // 256
    return m_tiles * ((N + 255) // 256) <= units // 2


def _full_rounds(M: int, N: int, E: int, device) -> bool:
    """True when the forward has at least one full round of 256x256 tiles for
    any group sizes and some group sizes could leave its last round at most
    half full.  Such a launch takes the split entry: the kernel cuts a last
    round that fills at most half of the units along K (at most 8 ranges) and
    leaves any other last round alone; the fixed-order reduction then costs
    one short launch.  The m-tile count lies between ceil(M / 256) and
    floor((M + 3(E-1) + 255 E) / 256) (see _small_launch), so a launch whose
    every possible tile count fills its last round more than half (one
    expert over whole rounds, for instance) skips that launch."""
    units = (_split_workspace_bytes(device) - 16384) // (256 * 256 * 4)
    n_tiles = (N + 255) // 256
    m_lo = (M + 255) // 256
    m_hi = max(m_lo, (M + 3 * (E - 1) + 255 * E) // 256)
    if m_lo * n_tiles < units:
        return False
    return any(0 < (m * n_tiles) % units <= units // 2 for m in range(m_lo, m_hi + 1))


_MAX_OPERAND_BYTES = 0x7FFFFFF0   # the C ABI's bound on (rows - 1) * ld + K


def _feature_rows_per_launch(ld: int, rows: int, M: int) -> int:
    """Feature rows of a token-axis wgrad operand [rows, M] (row stride ld
    bytes) one launch may take: all when it fits the 32-bit buffer range,
    else the largest multiple of 256 that does."""
    if rows == 0 or (rows - 1) * ld + M <= _MAX_OPERAND_BYTES:
        return max(rows, 1)
    return max(256, ((_MAX_OPERAND_BYTES - M) // ld + 1) // 256 * 256)


def _rows_per_launch(lda: int, K: int, M: int) -> int:
    """Rows of A one forward launch may take: all M when A fits the 32-bit
    buffer range, else the largest multiple of 256 that does."""
    if M == 0 or (M - 1) * lda + K <= _MAX_OPERAND_BYTES:
        return max(M, 1)
    return max(256, ((_MAX_OPERAND_BYTES - K) // lda + 1) // 256 * 256)


def grouped_mm(a: torch.Tensor, w: torch.Tensor, offs: torch.Tensor | None,
               a_scales: torch.Tensor | None = None, w_scales: torch.Tensor | None = None,
               out_dtype: torch.dtype = torch.bfloat16, out: torch.Tensor | None = None,
               split_tail: bool | None = None):
    """out[rows of g] = dequant(a[rows of g]) @ dequant(w[g])^T, fp32 accumulate.

    a: e4m3 [M, K]; w: e4m3 [E, N, K]; offs: int32 group ends ([E] or [E+1]
    with leading 0) or None for a single group; scales: E8M0 bytes
    [M, K/32] and [E, N, K/32], both or neither (neither = scale 1.0).
    Rows after the last group end are left untouched.  split_tail: run a
    launch whose tiles fill at most half of the compute units split along K
    over the idle units (mxgg_grouped_fwd_split; deterministic, equal to the
    unsplit result up to fp32 summation order).  None (default): when the
    launch is that small whatever the group sizes are, and when it has at
    least one full round of tiles and some group sizes could leave its last
    round at most half full (the kernel then splits that round only if it
    does); True: always take the split entry point; False: never.
    """
    _need_gpu(a, "a")
    _need_gpu(w, "w")
    if a.dim() != 2 or w.dim() != 3:
        raise ValueError(f"expected a [M, K] and w [E, N, K], got {tuple(a.shape)} and {tuple(w.shape)}")
    M, K = a.shape
    E, N, K2 = w.shape
    assert K == K2, f"K mismatch: {K} vs {K2}"
    a8 = _as_u8(_rowmajor(a), "a")
    w8 = _as_u8(_rowmajor(w), "w")
    if (a_scales is None) != (w_scales is None):
        raise ValueError("a_scales and w_scales must both be given or both be None")
    sa = sw = None
    ldas = ldws = wsg = 0
    if a_scales is not None:
        sa, ldas = _scales_2d(a_scales, M, K // 32, "a_scales")
        sw, wsg, ldws = _scales_3d(w_scales, E, N, K // 32, "w_scales")
    ends = None
    if offs is not None:
        ends = _group_ends(offs, E, a.device)
    elif E != 1:
        raise ValueError("offs is required when w holds more than one expert")
    padded = out is None and N % 4 != 0
    if padded:
        # the library writes rows at a stride of whole 4-element groups: a
        # column count off that grid runs into a wider buffer and is returned
        # as a contiguous copy
        out = torch.empty((M, (N + 3) // 4 * 4), dtype=out_dtype, device=a.device)[:, :N]
    elif out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    elif out.shape != (M, N) or out.dtype != out_dtype or out.stride(-1) != 1:
        raise ValueError("out must be a row-major [M, N] tensor of out_dtype")
    lib = _lib.load()
    stream = _stream_ptr(a)
    esz = out.element_size()
    rows = _rows_per_launch(a8.stride(0), K, M)
    for r0 in range(0, max(M, 1), rows):
        # Operands are read through 32-bit buffer ranges (< 2 GiB): a larger
        # activation matrix runs as row chunks (multiples of 256 rows), each
        # with the group ends shifted to the chunk and clamped to it (on the
        # device, no host sync).  Every output row still comes from one
        # full-K accumulation, so the chunked result is the same.
        m = min(rows, M - r0)
        e = ends
        if e is not None and rows < M:
            e = torch.clamp(ends - r0, 0, m)
        args = (a8.data_ptr() + r0 * a8.stride(0), a8.stride(0),
                sa.data_ptr() + r0 if sa is not None else None, ldas,
                w8.data_ptr(), w8.stride(0), w8.stride(1),
                sw.data_ptr() if sw is not None else None, wsg, ldws,
                e.data_ptr() if e is not None else None, E,
                m, N, K, out.data_ptr() + r0 * out.stride(0) * esz, out.stride(0),
                _out_code(out_dtype))
        split = (_small_launch(m, N, E, a.device) or _full_rounds(m, N, E, a.device)) \
            if split_tail is None else split_tail
        if split and m > 0 and N > 0:
            ws = _split_workspace(a.device)
            _lib.check(lib.mxgg_grouped_fwd_split(*args, ws.data_ptr(), ws.numel(), stream),
                       "grouped_fwd_split")
        else:
            _lib.check(lib.mxgg_grouped_fwd(*args, stream), "grouped_fwd")
    return out.contiguous() if padded else out


def grouped_mm_swiglu_quant(a: torch.Tensor, w: torch.Tensor, offs: torch.Tensor | None,
                            a_scales: torch.Tensor | None = None,
                            w_scales: torch.Tensor | None = None, scaling_mode="rceil",
                            return_h: bool = False):
    """The gate+up projection, SiLU(gate) * up and its row-wise MXFP8 cast in
    one kernel (mxgg_grouped_fwd_swiglu_quant).

    a: e4m3 [M, K]; w: e4m3 [E, 2F, K] with gate rows first (the fused gate+up
    weight); scales and offs as for grouped_mm.  F % 128 == 0.  Returns
    (q float8_e4m3fn [M, F], scales uint8 [M, F/32] view of block-major
    storage), equal to swiglu_quant(grouped_mm(a, w, ..., split_tail=False))
    on the rows inside the groups (rows past the last group end are not
    written; the fused kernel never splits K, so a launch that grouped_mm
    would split can differ from its default in the fp32 summation order).
    Without return_h the bf16 [M, 2F] projection is never materialised
    (forward-only passes); with it (the training forward,
    mxgg_grouped_fwd_swiglu_quant_keep_h) the kernel also writes
    h = grouped_mm(a, w, ..., split_tail=False) for the backward and returns
    (q, scales, h); rows of h past the last group end are zero.  The
    reference runs the gate and up GEMMs, eager SiLU * up and the fp8 cast
    separately (e2e_bench.py:56-61)."""
    _need_gpu(a, "a")
    _need_gpu(w, "w")
    if a.dim() != 2 or w.dim() != 3:
        raise ValueError(f"expected a [M, K] and w [E, 2F, K], got {tuple(a.shape)} and {tuple(w.shape)}")
    M, K = a.shape
    E, N2, K2 = w.shape
    if K != K2:
        raise ValueError(f"K mismatch: {K} vs {K2}")
    if N2 % 256 != 0:
        raise ValueError(f"w has {N2} rows; the fused path needs 2F with F % 128 == 0")
    F = N2 // 2
    a8 = _as_u8(_rowmajor(a), "a")
    w8 = _as_u8(_rowmajor(w), "w")
    if (a_scales is None) != (w_scales is None):
        raise ValueError("a_scales and w_scales must both be given or both be None")
    sa = sw = None
    ldas = ldws = wsg = 0
    if a_scales is not None:
        sa, ldas = _scales_2d(a_scales, M, K // 32, "a_scales")
        sw, wsg, ldws = _scales_3d(w_scales, E, N2, K // 32, "w_scales")
    ends = None
    if offs is not None:
        ends = _group_ends(offs, E, a.device)
    elif E != 1:
        raise ValueError("offs is required when w holds more than one expert")
    if M > 0 and (M - 1) * a8.stride(0) + K > _MAX_OPERAND_BYTES:
        raise ValueError("the fused SwiGLU forward takes activations below 2 GiB per call")
    q = torch.empty((M, F), dtype=_FP8, device=a.device)
    buf = _block_major_buffer(M, F // 32, a.device)
    lib = _lib.load()
    head = (a8.data_ptr(), a8.stride(0), sa.data_ptr() if sa is not None else None, ldas,
            w8.data_ptr(), w8.stride(0), w8.stride(1), sw.data_ptr() if sw is not None else None,
            wsg, ldws, ends.data_ptr() if ends is not None else None, E, M, F, K)
    tail = (q.data_ptr(), F, buf.data_ptr(), buf.stride(0), _lib.SCALES_BLOCK_MAJOR,
            _mode(scaling_mode), _stream_ptr(a))
    if not return_h:
        _lib.check(lib.mxgg_grouped_fwd_swiglu_quant(*head, *tail), "grouped_fwd_swiglu_quant")
        return q, buf[:, :M].t()
    # rows past the last group end are not written by the kernel: zero them
    # as the library's grouped_mm + zero_rows_past_groups would give
    h = torch.empty((M, 2 * F), dtype=torch.bfloat16, device=a.device)
    _lib.check(lib.mxgg_grouped_fwd_swiglu_quant_keep_h(*head, h.data_ptr(), 2 * F, *tail),
               "grouped_fwd_swiglu_quant_keep_h")
    if ends is not None:
        zero_rows_past_groups(h, ends)
    return q, buf[:, :M].t(), h


def fused_grouped_fwd(a_fp8, w_fp8, offs, a_scales=None, w_scales=None,
                      BLOCK_M=128, BLOCK_N=128, BLOCK_K=128,
                      GROUP_SIZE_M=8, num_stages=None, num_warps=None, *,
                      out_dtype=torch.bfloat16):
    """Drop-in for fused_fwd.fused_grouped_fwd (fused_fwd.py:172-229).

    a_fp8 [M, K] e4m3, w_fp8 [E, N, K] e4m3, offs group ends (honoured, also
    when groups are unequal or empty), optional E8M0 scales [M, K/32] and
    [E, N, K/32].  As in the reference, scales are used only when both are
    given.  The tile keyword arguments are accepted for call-site
    compatibility; the gfx950 kernel uses its own fixed 256x256x128 tiling.
    Returns bf16 [M, N].
    """
    del BLOCK_M, BLOCK_N, BLOCK_K, GROUP_SIZE_M, num_stages, num_warps
    use_scales = a_scales is not None and w_scales is not None
    return grouped_mm(a_fp8, w_fp8, offs,
                      a_scales if use_scales else None, w_scales if use_scales else None,
                      out_dtype=out_dtype)


def fwd_ge(x_fp8, w_fp8, BLOCK_M=256, BLOCK_N=256, BLOCK_K=128, NUM_WARPS=4, GROUP_M=4):
    """Drop-in for fwd_final.fwd_ge (fwd_final.py:121-131): C[M,N] = X[M,K] @ W[K,N].

    Unscaled (every E8M0 scale 1.0), bf16 out.  W [K, N] is consumed as its
    transpose [N, K]; a W that is itself a transposed view of a row-major
    [N, K] tensor (the layout the reference transposes away from,
    fwd_final.py:189) is used without a copy.
    """
    del BLOCK_M, BLOCK_N, BLOCK_K, NUM_WARPS, GROUP_M
    M, K = x_fp8.shape
    K2, N = w_fp8.shape
    assert K == K2
    wt = w_fp8.t()
    if wt.stride(-1) != 1:
        wt = wt.contiguous()
    return grouped_mm(x_fp8, wt.unsqueeze(0), None)


# ---------------------------------------------------------------------------
# wgrad grouped GEMM
# ---------------------------------------------------------------------------
def _cu_count(device) -> int:
    return torch.cuda.get_device_properties(device).multi_processor_count


def wgrad_split_tokens(M: int, N: int, K: int, E: int, cus: int) -> int:
    """Split-K chunk (tokens) for a weight-gradient call, from shapes only.

    With at most cus/2 output tiles (E * ceil(N/256) * ceil(K/256)) most
    compute units would idle, so each expert's tokens are cut into up to
    min(16, cus/tiles) chunks of at least 4096 tokens: about one round of
    work items, each writing an fp32 partial tile that a second kernel adds in
    chunk order (measured best on 32, 64 and 128 tiles; with more tiles the
    partials cost more than the idle units).  The M tokens are assumed to
    spread evenly over the experts (group sizes live on the device and are not
    read back).  Returns 0 for no split."""
    tiles = E * ((N + 255) // 256) * ((K + 255) // 256)
    if tiles == 0 or M == 0 or 2 * tiles > cus:
        return 0
    per_expert = max(1, M // max(E, 1))
    splits = min(16, cus // tiles)
    chunk = max(4096, (per_expert + splits - 1) // splits)
    chunk = (chunk + 127) // 128 * 128
    return 0 if chunk >= per_expert else chunk


def grouped_wgrad(go: torch.Tensor, ia: torch.Tensor, offs: torch.Tensor,
                  go_scales: torch.Tensor | None = None, ia_scales: torch.Tensor | None = None,
                  out_dtype: torch.dtype = torch.float32, out: torch.Tensor | None = None,
                  split_tokens: int | None = None):
    """dW[g] = dequant(go[:, tok of g]) @ dequant(ia[:, tok of g])^T  -> [E, N, K].

    go: e4m3 [N, M] (dY transposed, token-contiguous); ia: e4m3 [K, M]
    (X transposed); offs: int32 [E] cumulative token ends; scales: E8M0
    [N, M/32] / [K, M/32] along tokens, both or neither.  With scales every
    group end must be a multiple of 32 (the layout to_mxfp8_dim1 produces): an
    expert whose bounds are not is written as NaN, since a scale block would
    span two experts.  Without scales the ends may be any token index.
    Empty groups yield zeros.  An operand past the 2 GiB buffer range of one
    launch (e.g. X^T at K = 7168 from 299593 tokens) runs as launches over
    chunks of its feature rows, each writing its slice of dW.
    split_tokens: split-K chunk in tokens (multiple of 128), 0 for none, None
    to choose from the shapes (wgrad_split_tokens).  A split call writes the
    fp32 partial tiles to a workspace and adds them in chunk order
    (mxgg_grouped_wgrad_split): deterministic, any output dtype, equal to the
    unsplit result up to fp32 summation order.
    """
    _need_gpu(go, "go")
    _need_gpu(ia, "ia")
    if go.dim() != 2 or ia.dim() != 2:
        raise ValueError("go and ia must be 2-D")
    N, M = go.shape
    K, M2 = ia.shape
    assert M == M2, f"token count mismatch: {M} vs {M2}"
    g8 = _as_u8(_rowmajor(go), "go")
    i8 = _as_u8(_rowmajor(ia), "ia")
    if (go_scales is None) != (ia_scales is None):
        raise ValueError("go_scales and ia_scales must both be given or both be None")
    sg = si = None
    ldgs = ldis = 0
    if go_scales is not None:
        sg, ldgs = _scales_2d(go_scales, N, M // 32, "go_scales")
        si, ldis = _scales_2d(ia_scales, K, M // 32, "ia_scales")
    E = offs.numel()
    ends = _group_ends(offs, E, go.device)
    padded = out is None and K % 4 != 0
    if padded:
        # dW rows at a stride of whole 4-element groups (the strided entry),
        # returned as a contiguous copy
        out = torch.empty((E, N, (K + 3) // 4 * 4), dtype=out_dtype, device=go.device)[:, :, :K]
    elif out is None:
        out = torch.empty((E, N, K), dtype=out_dtype, device=go.device)
    elif out.shape != (E, N, K) or out.dtype != out_dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous [E, N, K] tensor of out_dtype")
    lib = _lib.load()
    nc = _feature_rows_per_launch(g8.stride(0), N, M)
    kc = _feature_rows_per_launch(i8.stride(0), K, M)
    if nc < N or kc < K or padded:
        # An operand past the 32-bit buffer range: launches over chunks of its
        # feature rows (256-row multiples), each contracting every token and
        # writing its own slice of dW (mxgg_grouped_wgrad_strided), so the
        # result is the one-launch result.  A padded dW goes the same way
        # (one chunk each way) for its row stride.
        esz = out.element_size()
        for n0 in range(0, N, nc):
            for k0 in range(0, K, kc):
                n, k = min(nc, N - n0), min(kc, K - k0)
                st = wgrad_split_tokens(M, n, k, E, _cu_count(go.device)) \
                    if split_tokens is None else int(split_tokens)
                ws, nbytes = None, 0
                if st:
                    nbytes = int(lib.mxgg_grouped_wgrad_workspace_bytes(M, n, k, E, st))
                    if nbytes < 0:
                        raise ValueError(f"split_tokens={st} must be a positive multiple of 128")
                    ws = torch.empty(nbytes, dtype=torch.uint8, device=go.device)
                _lib.check(lib.mxgg_grouped_wgrad_strided(
                    g8.data_ptr() + n0 * g8.stride(0), g8.stride(0),
                    sg.data_ptr() + n0 if sg is not None else None, ldgs,
                    i8.data_ptr() + k0 * i8.stride(0), i8.stride(0),
                    si.data_ptr() + k0 if si is not None else None, ldis,
                    ends.data_ptr(), E, M, n, k,
                    out.data_ptr() + (n0 * out.stride(1) + k0) * esz, out.stride(0),
                    out.stride(1), _out_code(out_dtype), st,
                    ws.data_ptr() if ws is not None else None, nbytes, _stream_ptr(go)),
                    "grouped_wgrad_strided")
        return out.contiguous() if padded else out
    if split_tokens is None:
        split_tokens = wgrad_split_tokens(M, N, K, E, _cu_count(go.device))
    args = (g8.data_ptr(), g8.stride(0),
            sg.data_ptr() if sg is not None else None, ldgs,
            i8.data_ptr(), i8.stride(0),
            si.data_ptr() if si is not None else None, ldis,
            ends.data_ptr(), E, M, N, K, out.data_ptr(), _out_code(out_dtype), int(split_tokens))
    if split_tokens:
        nbytes = int(lib.mxgg_grouped_wgrad_workspace_bytes(M, N, K, E, int(split_tokens)))
        if nbytes < 0:
            raise ValueError(f"split_tokens={split_tokens} must be a positive multiple of 128")
        ws = torch.empty(nbytes, dtype=torch.uint8, device=go.device)
        _lib.check(lib.mxgg_grouped_wgrad_split(*args, ws.data_ptr(), nbytes, _stream_ptr(go)),
                   "grouped_wgrad_split")
    else:
        _lib.check(lib.mxgg_grouped_wgrad(*args, _stream_ptr(go)), "grouped_wgrad")
    return out


def _best_config(e, m):
    """Reference tile heuristic (wgrad_fused.py:22-31).  Kept for call-site
    compatibility; the gfx950 kernel ignores tile hints."""
    if m >= 100000:
        return dict(BLOCK_M=256, BLOCK_N=256, BLOCK_K=128, GROUP_SIZE_M=4,
                    num_stages=None, num_warps=4)
    return dict(BLOCK_M=128, BLOCK_N=128, BLOCK_K=128, GROUP_SIZE_M=1,
                num_stages=2 if e <= 4 else None, num_warps=4)


_TILE_KW = ("BLOCK_M", "BLOCK_N", "BLOCK_K", "GROUP_SIZE_M", "num_stages", "num_warps")


def _split_kw(kwargs):
    out_dtype = kwargs.pop("out_dtype", torch.bfloat16)
    for k in list(kwargs):
        if k in _TILE_KW:
            kwargs.pop(k)
    if kwargs:
        raise TypeError(f"unexpected keyword arguments: {sorted(kwargs)}")
    return out_dtype


def _wgrad_offs(offs, tokens: int, offs_kind: str, device):
    if not isinstance(offs, torch.Tensor):
        offs = torch.as_tensor(offs, dtype=torch.int32)
    if offs.dim() != 1 or offs.numel() < 1:
        raise ValueError(f"offs must be a non-empty 1-D tensor, got shape {tuple(offs.shape)}")
    if offs.device != device:
        offs = offs.to(device, non_blocking=True)   # a GroupEnds stays one
    return offs_to_group_ends(offs, tokens, offs_kind)


def wgrad_fused(go, ia, offs, go_scales=None, ia_scales=None, *, offs_kind="auto", **kwargs):
    """Drop-in for wgrad_fused.wgrad_fused (wgrad_fused.py:34-71).

    go (N, M) e4m3, ia (K, M) e4m3, offs (E,) int32, optional E8M0 scales
    (N, M/32) and (K, M/32).  The reference documents offs as group sizes
    (wgrad_fused.py:37; bench_wgrad_dsv3.py:52 passes [M/E] * E) while its
    layer step passes cumulative ends (e2e_bench.py:42,117); it reads neither
    and splits M // E tokens per expert.  Here the groups are honoured: with
    offs_kind="auto" (default) offs is read as sizes when its entries add up
    to exactly M and its last entry is below M, as cumulative ends otherwise;
    "sizes" / "ends" force one reading (offs_to_group_ends).  Group ends from
    this library's token-axis casts (GroupEnds) are always read as ends.  No restacking:
    the kernel contracts each group's token range in place.  Returns
    (E, N, K), bf16 by default like the reference; pass
    out_dtype=torch.float32 for fp32 grads.  Scales are used only when both
    are given, as in the reference.
    """
    out_dtype = _split_kw(dict(kwargs))
    _need_gpu(go, "go")
    use_scales = go_scales is not None and ia_scales is not None
    ends = _wgrad_offs(offs, go.shape[1], offs_kind, go.device)
    return grouped_wgrad(go, ia, ends, go_scales if use_scales else None,
                         ia_scales if use_scales else None, out_dtype=out_dtype)


def wgrad_prepare(go, ia, offs, go_scales=None, ia_scales=None, *, offs_kind="auto"):
    """Drop-in for wgrad_fused.wgrad_prepare (wgrad_fused.py:74-103).

    The reference restacks per group here; this kernel needs no restacking,
    so the dict references the caller's tensors (same keys as the reference).
    "offs" holds the cumulative group ends read from `offs` as wgrad_fused
    reads it (sizes or ends, see there).
    """
    _need_gpu(go, "go")
    N, M = go.shape
    K = ia.shape[0]
    E = offs.shape[0]
    use_scales = go_scales is not None and ia_scales is not None
    return {
        "A": go, "B": ia,
        "offs": _wgrad_offs(offs, M, offs_kind, go.device),
        "As": go_scales if use_scales else None, "Bs": ia_scales if use_scales else None,
        "E": E, "N": N, "K": K, "M": M,
        "flops": 2 * M * N * K,
    }


def wgrad_kernel(data: dict, **kwargs):
    """Drop-in for wgrad_fused.wgrad_kernel (wgrad_fused.py:106-112): run on a
    wgrad_prepare() dict, return (E, N, K) (bf16 unless out_dtype is given)."""
    out_dtype = _split_kw(dict(kwargs))
    return grouped_wgrad(data["A"], data["B"], data["offs"], data["As"], data["Bs"],
                         out_dtype=out_dtype)


# ---------------------------------------------------------------------------
# data gradient  dX = dY . W  (MXFP8 blocks along N)
# ---------------------------------------------------------------------------
def quant_weight_for_dgrad(w: torch.Tensor, scaling_mode="rceil"):
    """W [E, N, K] bf16 -> W_e^T quantised with 1x32 blocks along N, for dgrad.

    Runs the token-axis cast on W viewed as [E*N, K] with one group per
    expert, so expert e's transposed weights are columns [e*N, (e+1)*N) of a
    [K, E*N] e4m3 matrix.  Returns (wt, wts): wt a strided e4m3 view
    [E, K, N] and wts an E8M0 view [E, K, N/32] of block-major storage, both
    ready for grouped_mm.  N must be a multiple of 32 (no block may straddle
    two experts).  Weights change only at the optimizer step, so a trainer
    computes this once per step for the whole backward pass.
    """
    _need_gpu(w, "w")
    if w.dtype != torch.bfloat16 or w.dim() != 3:
        raise TypeError("w must be a 3-D bfloat16 tensor [E, N, K]")
    E, N, K = w.shape
    if N % 32 != 0:
        raise ValueError(f"N={N} must be a multiple of 32 for MXFP8 blocks along N")
    qt, st, _ = to_mxfp8_dim1(w.reshape(E * N, K), _expert_ends(E, N, w.device), scaling_mode)
    return _weight_t_views(qt, st, E, N, K)


def grouped_dgrad(dy: torch.Tensor, w: torch.Tensor | tuple, offs: torch.Tensor,
                  out_dtype: torch.dtype = torch.bfloat16, scaling_mode="rceil",
                  out: torch.Tensor | None = None):
    """dX[rows of g] = dY[rows of g] . W[g] with MXFP8 operands blocked along N.

    dy: bf16 [M, N] (gradient of the layer output); w: bf16 [E, N, K] or the
    (wt, wts) pair from quant_weight_for_dgrad; offs: token group ends as for
    grouped_mm.  dY is cast along N (dim0), W_e^T along N, and the product
    runs on the forward grouped GEMM (contraction over N).  Returns [M, K].
    (The reference computes this step in bf16 per expert, e2e_bench.py:91-108.)
    """
    _need_gpu(dy, "dy")
    if dy.dtype != torch.bfloat16 or dy.dim() != 2:
        raise TypeError("dy must be a 2-D bfloat16 tensor [M, N]")
    wt, wts = w if isinstance(w, tuple) else quant_weight_for_dgrad(w, scaling_mode)
    dyq, dys = to_mxfp8_dim0(dy, scaling_mode)
    return grouped_mm(dyq, wt, offs, dys, wts, out_dtype=out_dtype, out=out)
