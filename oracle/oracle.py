"""CPU oracle for the MXFP8 grouped-GEMM path.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, always as the checker; the product
(mxfp8gg / libmxgg.so) never imports or calls anything here.

Pieces (reference paths under /root/reference):
  * quantisation: mx_oracle.c (ctypes) — e4m3 RNE table search, E8M0
    RCEIL/FLOOR from double-precision frexp, dim0 and grouped dim1 casts.
  * grouped forward reference: dequantise, then per-group matmul in float64,
    grouped semantics of reference_grouped_gemm (fused_fwd.py:249-264:
    rows [offs[g-1], offs[g]) use W[g]; empty groups are skipped) with the
    dequantisation of scale_correctness.py:112-137 (value * 2^(b-127)).
  * wgrad reference: dW[g] = dY_g^T X_g over each group's tokens
    (wgrad_fused.py:4 docstring, e2e_bench.py:113-131), empty group -> 0.
  * cpu_baseline_*: the same dequant + per-group matmul in float32 with torch
    on all host cores — the reference's torch CPU dequant path, timed by
    bench.py as the CPU baseline.
  * swiglu_fwd / swiglu_bwd: the expert FFN activation a = SiLU(gate) * up
    and its gradients in float32 with bf16 rounding after each op, the eager
    bf16 torch arithmetic of the reference's layer step (e2e_bench.py:56-61,
    85-100) with the textbook SiLU derivative sig * (1 + g * (1 - sig)).
  * route_plan / gather_rows / combine / combine_score_grad: the token
    dispatch and combine around the expert GEMMs that the reference takes
    from torchtitan's token dispatcher with pad_multiple = 32
    (port_mxfp8.py:214, 240): slots s = t * topk + k grouped by expert in
    slot order (a sequential counting sort here), groups padded with empty
    rows, routed input x[s // topk], combine = sum over k of the routed
    output times its score (rounded to bf16), summed in float32 in k order.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "mx_oracle.c"
LIB = HERE / "liboracle.so"

RCEIL = 0
FLOOR = 1


def build() -> Path:
    """Compile mx_oracle.c into liboracle.so (plain gcc, no GPU)."""
    tmp = LIB.with_suffix(".so.tmp")
    subprocess.run(["gcc", "-O2", "-shared", "-fPIC", "-Wall", "-o", str(tmp), str(SRC), "-lm"],
                   check=True)
    tmp.replace(LIB)
    return LIB


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists() or LIB.stat().st_mtime < SRC.stat().st_mtime:
            build()
        L = ctypes.CDLL(str(LIB))
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.mxo_e4m3_decode.restype = ctypes.c_double
        L.mxo_e4m3_decode.argtypes = [ctypes.c_uint8]
        L.mxo_e4m3_encode.restype = ctypes.c_uint8
        L.mxo_e4m3_encode.argtypes = [ctypes.c_double]
        L.mxo_e8m0.restype = ctypes.c_uint8
        L.mxo_e8m0.argtypes = [ctypes.c_double, I]
        L.mxo_payload.restype = ctypes.c_uint8
        L.mxo_payload.argtypes = [ctypes.c_double, ctypes.c_uint8, I]
        L.mxo_quant_dim0.restype = None
        L.mxo_quant_dim0.argtypes = [P, I64, I64, P, P, I]
        L.mxo_quant_dim1.restype = None
        L.mxo_quant_dim1.argtypes = [P, I64, I64, P, I64, I64, P, P, P, I]
        L.mxo_dequant.restype = None
        L.mxo_dequant.argtypes = [P, P, I64, I64, I64, I64, P]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# ---------------------------------------------------------------------------
# scalar rules
# ---------------------------------------------------------------------------
E4M3_TABLE = None


def e4m3_table() -> np.ndarray:
    """float64 value of each of the 256 e4m3fn codes (NaN for 0x7F / 0xFF)."""
    global E4M3_TABLE
    if E4M3_TABLE is None:
        L = lib()
        E4M3_TABLE = np.array([L.mxo_e4m3_decode(c) for c in range(256)], dtype=np.float64)
    return E4M3_TABLE


def e4m3_encode(v: float) -> int:
    return int(lib().mxo_e4m3_encode(float(v)))


def e8m0(amax: float, mode: int = RCEIL) -> int:
    return int(lib().mxo_e8m0(float(amax), mode))


def payload(x: float, b: int, mode: int = RCEIL) -> int:
    return int(lib().mxo_payload(float(x), b, mode))


# ---------------------------------------------------------------------------
# casts (bf16 given as its uint16 bit pattern)
# ---------------------------------------------------------------------------
def quant_dim0(x_bits: np.ndarray, mode: int = RCEIL):
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    R, C = x.shape
    assert C % 32 == 0
    q = np.empty((R, C), np.uint8)
    s = np.empty((R, C // 32), np.uint8)
    lib().mxo_quant_dim0(_ptr(x), R, C, _ptr(q), _ptr(s), mode)
    return q, s


def quant_dim1(x_bits: np.ndarray, ends: np.ndarray | None, cap: int, mode: int = RCEIL):
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    R, C = x.shape
    qt = np.empty((C, cap), np.uint8)
    st = np.empty((C, cap // 32), np.uint8)
    if ends is None:
        lib().mxo_quant_dim1(_ptr(x), R, C, None, 0, cap, _ptr(qt), _ptr(st), None, mode)
        return qt, st, None
    e = np.ascontiguousarray(ends, dtype=np.int32)
    pad = np.empty(e.shape[0], np.int32)
    lib().mxo_quant_dim1(_ptr(x), R, C, _ptr(e), e.shape[0], cap, _ptr(qt), _ptr(st), _ptr(pad),
                         mode)
    return qt, st, pad


def dequant(q: np.ndarray, s: np.ndarray | None) -> np.ndarray:
    """float64 values of e4m3 payload q [..., K] with E8M0 scales s [..., K/32]."""
    vals = e4m3_table()[q]
    if s is None:
        return vals
    sc = np.where(s == 255, np.nan, np.ldexp(1.0, s.astype(np.int64) - 127))
    return vals * np.repeat(sc, 32, axis=-1)


def group_bounds(ends, rows: int):
    """[(beg, end)] per group under the library's documented rule for group
    ends: m[g] = the running maximum of ends[0..g] clamped to [0, rows], group
    g = [m[g-1], m[g]) with m[-1] = 0 (well-formed non-decreasing ends are used
    as given; a decreasing entry gives an empty group)."""
    out = []
    m_prev = 0
    for e in np.asarray(ends).tolist():
        m = min(max(m_prev, e, 0), rows)
        out.append((m_prev, m))
        m_prev = m
    return out


def rows_in_groups(ends, rows: int) -> np.ndarray:
    """Boolean mask over `rows` rows: True for the rows that belong to a group
    under group_bounds (the rows a grouped forward writes)."""
    mask = np.zeros(rows, dtype=bool)
    for b, e in group_bounds(ends, rows):
        mask[b:e] = True
    return mask


# ---------------------------------------------------------------------------
# GEMM references (float64)
# ---------------------------------------------------------------------------
def grouped_fwd(a_q, a_s, w_q, w_s, ends, rows=None):
    """Y[rows of g] = dequant(A)[rows of g] @ dequant(W[g])^T in float64.

    Rows outside every group are NaN (the kernel leaves them untouched).
    `rows` optionally restricts the computation to a sorted subset of rows
    (returned in that order) for sampled checks at full size."""
    M, K = a_q.shape
    E, N, _ = w_q.shape
    bounds = group_bounds(ends, M) if ends is not None else [(0, M)]
    rows = np.arange(M) if rows is None else np.asarray(rows)
    out = np.full((rows.shape[0], N), np.nan)
    for g, (b, e) in enumerate(bounds):
        sel = np.nonzero((rows >= b) & (rows < e))[0]
        if sel.size == 0:
            continue
        a = dequant(a_q[rows[sel]], None if a_s is None else a_s[rows[sel]])
        w = dequant(w_q[g], None if w_s is None else w_s[g])
        out[sel] = a @ w.T
    return out


def grouped_wgrad(go_q, go_s, ia_q, ia_s, ends, n_rows=None, k_rows=None):
    """dW[g] = dequant(go)[:, tok g] @ dequant(ia)[:, tok g]^T, float64 [E, n, k].
    n_rows / k_rows optionally select output rows / columns."""
    N, M = go_q.shape
    K, _ = ia_q.shape
    n_rows = np.arange(N) if n_rows is None else np.asarray(n_rows)
    k_rows = np.arange(K) if k_rows is None else np.asarray(k_rows)
    bounds = group_bounds(ends, M)
    out = np.zeros((len(bounds), n_rows.shape[0], k_rows.shape[0]))
    go = dequant(go_q[n_rows], None if go_s is None else go_s[n_rows])
    ia = dequant(ia_q[k_rows], None if ia_s is None else ia_s[k_rows])
    for g, (b, e) in enumerate(bounds):
        if e > b:
            out[g] = go[:, b:e] @ ia[:, b:e].T
    return out


# ---------------------------------------------------------------------------
# CPU baseline: the reference's torch CPU dequant path, float32, all cores
# ---------------------------------------------------------------------------
def cpu_baseline_fwd(a_q, a_s, w_q, w_s, ends):
    """torch float32 on CPU: dequantise then per-group matmul (timed by bench.py)."""
    import torch

    table = torch.from_numpy(e4m3_table().astype(np.float32))

    def deq(q, s):
        v = table[q.long()]
        sc = torch.pow(2.0, s.float() - 127.0).repeat_interleave(32, dim=-1)
        return v * sc

    M = a_q.shape[0]
    out = torch.empty((M, w_q.shape[1]), dtype=torch.float32)
    for g, (b, e) in enumerate(group_bounds(ends.tolist(), M)):
        if e > b:
            out[b:e] = deq(a_q[b:e], a_s[b:e]) @ deq(w_q[g], w_s[g]).T
    return out


# ---------------------------------------------------------------------------
# SwiGLU (expert FFN activation), bf16 in / bf16 out, float32 arithmetic
# ---------------------------------------------------------------------------
def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 (ties to even), returned as float32 values."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), np.float32(np.nan), r).astype(np.float32)


def bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bits(x: np.ndarray) -> np.ndarray:
    """bf16-representable float32 values -> uint16 bit patterns."""
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def swiglu_fwd(g_bits: np.ndarray, u_bits: np.ndarray) -> np.ndarray:
    """a = bf16(bf16(g / (1 + exp(-g))) * u) (torch's eager bf16 F.silu(g) * u)."""
    g = bits_to_f32(g_bits)
    u = bits_to_f32(u_bits)
    with np.errstate(over="ignore", invalid="ignore"):
        s = bf16_round(g / (np.float32(1) + np.exp(-g)))
        return f32_to_bits(bf16_round(s * u))


def swiglu_bwd(g_bits: np.ndarray, u_bits: np.ndarray, d_bits: np.ndarray):
    """Gradients of a = silu(g) * u for upstream d = dL/da, as torch's eager
    bf16 autograd computes them:
      d_up   = bf16(d * s),  s = bf16(silu(g))
      d_gate = bf16(bf16(d * u) * sig * (1 + g * (1 - sig))),  sig = 1/(1+exp(-g))
    Returns (a, d_gate, d_up) as bf16 bit patterns."""
    g = bits_to_f32(g_bits)
    u = bits_to_f32(u_bits)
    d = bits_to_f32(d_bits)
    one = np.float32(1)
    with np.errstate(over="ignore", invalid="ignore"):
        ex = np.exp(-g)
        s = bf16_round(g / (one + ex))
        sig = one / (one + ex)
        ds = bf16_round(d * u)
        dg = bf16_round(ds * sig * (one + g * (one - sig)))
        du = bf16_round(d * s)
        a = bf16_round(s * u)
    return f32_to_bits(a), f32_to_bits(dg), f32_to_bits(du)


# ---------------------------------------------------------------------------
# Token routing of a top-k MoE layer (dispatch plan, gather, combine)
# ---------------------------------------------------------------------------
def route_plan(expert_idx: np.ndarray, num_experts: int, pad_multiple: int, rows_cap: int):
    """Sequential counting sort of the slots s = t * topk + k by expert.

    Returns (perm [n] int32: row of each slot, -1 for ids outside
    [0, num_experts); src [rows_cap] int32: slot of each row, -1 for padding;
    ends [E] int32: cumulative group ends, each group padded to a multiple of
    pad_multiple; counts [E] int32)."""
    idx = np.asarray(expert_idx, dtype=np.int64).reshape(-1)
    E = int(num_experts)
    counts = np.zeros(E, dtype=np.int64)
    for e in idx:
        if 0 <= e < E:
            counts[e] += 1
    padded = (counts + pad_multiple - 1) // pad_multiple * pad_multiple
    ends = np.cumsum(padded)
    nxt = ends - padded
    perm = np.full(idx.size, -1, dtype=np.int32)
    src = np.full(rows_cap, -1, dtype=np.int32)
    for s, e in enumerate(idx):
        if 0 <= e < E:
            r = nxt[e]
            nxt[e] += 1
            perm[s] = r
            src[r] = s
    return perm, src, ends.astype(np.int32), counts.astype(np.int32)


def gather_rows(x_bits: np.ndarray, src: np.ndarray, topk: int, row_scale=None) -> np.ndarray:
    """Routed rows (bf16 bits): x[src // topk], times row_scale[src] rounded to
    bf16 when given; zero rows where src < 0 or the token is out of range."""
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    out = np.zeros((src.size, x_bits.shape[1]), dtype=np.uint16)
    tok = np.where(src >= 0, src // topk, -1)
    ok = (tok >= 0) & (tok < x_bits.shape[0])
    rows = x_bits[tok[ok]]
    if row_scale is not None:
        sc = np.asarray(row_scale, dtype=np.float32).reshape(-1)[src[ok]]
        rows = f32_to_bits(bf16_round(bits_to_f32(rows) * sc[:, None]))
    out[ok] = rows
    return out


def combine(y_bits: np.ndarray, perm: np.ndarray, topk: int, scores=None) -> np.ndarray:
    """out[t] = bf16(sum_k term_k) (bf16 bits) summed in float32, k = 0, 1, ...,
    with term_k = bf16(float(y[perm[s]]) * score[s]) (the row itself without
    scores); slots with perm < 0 add nothing."""
    y_bits = np.asarray(y_bits, dtype=np.uint16)
    p = np.asarray(perm).reshape(-1, topk)
    T, H = p.shape[0], y_bits.shape[1]
    acc = np.zeros((T, H), dtype=np.float32)
    for k in range(topk):
        r = p[:, k]
        ok = (r >= 0) & (r < y_bits.shape[0])
        term = np.zeros((T, H), dtype=np.float32)
        term[ok] = bits_to_f32(y_bits[r[ok]])
        if scores is not None:
            sc = np.asarray(scores, dtype=np.float32).reshape(T, topk)[:, k]
            term = bf16_round(term * sc[:, None])
        acc = (acc + term).astype(np.float32)
    return f32_to_bits(bf16_round(acc))


def combine_score_grad(dout_bits: np.ndarray, y_bits: np.ndarray, perm: np.ndarray,
                       topk: int) -> np.ndarray:
    """d score[s] = sum_h dout[t][h] * y[perm[s]][h] (float64), 0 for dropped slots."""
    d = bits_to_f32(np.asarray(dout_bits, dtype=np.uint16)).astype(np.float64)
    y = bits_to_f32(np.asarray(y_bits, dtype=np.uint16)).astype(np.float64)
    p = np.asarray(perm).reshape(-1, topk)
    out = np.zeros(p.shape, dtype=np.float64)
    for k in range(topk):
        r = p[:, k]
        ok = (r >= 0) & (r < y.shape[0])
        out[ok, k] = np.einsum("th,th->t", d[ok], y[r[ok]])
    return out
