"""Pins the CPU oracle (oracle/) before it is trusted as the GPU checker.

Each check is independent of the oracle's own formulas:
  * e4m3: against torch's CPU float8_e4m3fn cast (an independent RNE
    implementation) on every bf16 pattern, every tie point and random fp32;
  * E8M0: against brute-force searches over candidate exponents written from
    the rule's definition (smallest power covering amax/448; largest power
    below amax);
  * GEMM: against the reference's known answers (scale_correctness.py:228,
    :310, :391), against pure-Python loops on tiny inputs, and the exact
    power-of-two scaling invariant;
  * dim1: against the transposed dim0 cast of each zero-padded group.
  * routing: against a hand-worked plan, torch's stable argsort of the expert
    ids (the dispatcher's own formula), torch's index ops for the gather and
    combine, and torch autograd for the combine's score gradient.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------------------
# e4m3 payload encoding
# ---------------------------------------------------------------------------
def torch_e4m3(vals_f32: np.ndarray) -> np.ndarray:
    return torch.from_numpy(vals_f32.astype(np.float32)).to(torch.float8_e4m3fn).view(
        torch.uint8).numpy()


def test_e4m3_decode_matches_torch():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().double().numpy()
    got = O.e4m3_table()
    assert np.array_equal(np.isnan(ref), np.isnan(got))
    ok = ~np.isnan(ref)
    assert np.array_equal(ref[ok], got[ok])


def _enc(vals):
    return np.array([O.e4m3_encode(v) for v in vals], dtype=np.uint8)


def test_e4m3_encode_all_bf16_patterns():
    bits = np.arange(65536, dtype=np.uint32) << 16
    vals = bits.view(np.float32)
    with np.errstate(invalid="ignore"):  # the sweep includes every NaN pattern
        got = _enc(vals.astype(np.float64))
    ref = torch_e4m3(vals)
    assert np.array_equal(got, ref)


def test_e4m3_encode_ties_and_neighbours():
    table = O.e4m3_table()
    pos = np.sort(table[:127])
    mids = (pos[:-1] + pos[1:]) / 2.0  # exact tie points (representable in fp32)
    vals = []
    for m in mids.astype(np.float32):
        vals += [np.nextafter(m, np.float32(-1)), m, np.nextafter(m, np.float32(1e9))]
    vals = np.array(vals + [464.0, 464.0001, 479.99, 480.0, 1e30, -464.0, 2.0 ** -10,
                            2.0 ** -10 * 1.0001, 2.0 ** -11], dtype=np.float32)
    vals = np.concatenate([vals, -vals])
    assert np.array_equal(_enc(vals.astype(np.float64)), torch_e4m3(vals))


def test_e4m3_encode_random_fp32():
    rng = np.random.default_rng(0)
    vals = (rng.standard_normal(20000) * np.exp2(rng.integers(-14, 9, 20000))).astype(np.float32)
    assert np.array_equal(_enc(vals.astype(np.float64)), torch_e4m3(vals))


# ---------------------------------------------------------------------------
# E8M0 scale rules
# ---------------------------------------------------------------------------
def _bf16_nonneg_finite():
    bits = np.arange(0, 0x7F80, dtype=np.uint32) << 16
    return bits.view(np.float32).astype(np.float64)


def brute_rceil(amax: float) -> int:
    """Smallest c in [-127, 127] with 448 * 2^c >= amax (c = -127 if amax is tiny)."""
    for c in range(-127, 128):
        if math.ldexp(448.0, c) >= amax:
            return c + 127
    return 254


def brute_floor(amax: float) -> int:
    """floor(log2 amax) by search, fp32-subnormal amax counted as exponent -127."""
    if amax < 2.0 ** -126:
        f = -127
    else:
        f = max(e for e in range(-126, 129) if 2.0 ** e <= amax)
    return min(max(f - 8, -127), 128) + 127


def test_e8m0_rceil_exhaustive_bf16():
    vals = _bf16_nonneg_finite()
    got = np.array([O.e8m0(v, O.RCEIL) for v in vals])
    ref = np.array([0 if v == 0 else brute_rceil(v) for v in vals])
    assert np.array_equal(got, ref)


def test_e8m0_floor_exhaustive_bf16():
    vals = _bf16_nonneg_finite()
    got = np.array([O.e8m0(v, O.FLOOR) for v in vals])
    ref = np.array([0 if v == 0 else brute_floor(v) for v in vals])
    assert np.array_equal(got, ref)


def test_e8m0_specials():
    assert O.e8m0(float("nan"), O.RCEIL) == 255
    assert O.e8m0(float("nan"), O.FLOOR) == 255
    assert O.e8m0(float("inf"), O.RCEIL) == 254
    assert O.e8m0(float("inf"), O.FLOOR) == 247
    assert O.e8m0(448.0, O.RCEIL) == 127           # amax/448 = 1 exactly
    assert O.e8m0(448.0 * 2 ** 5, O.RCEIL) == 132
    assert O.e8m0(449.0, O.RCEIL) == 128
    assert O.e8m0(1.0, O.FLOOR) == 119             # 2^0 / 2^8


def test_rceil_payload_of_block_max_is_in_top_binade():
    # RCEIL maps the block max into (224, 448]; FLOOR into [256, 512) before clamping.
    rng = np.random.default_rng(1)
    for v in np.abs(rng.standard_normal(2000)) * np.exp2(rng.integers(-40, 40, 2000)):
        v = float(np.float32(v))
        b = O.e8m0(v, O.RCEIL)
        y = O.e4m3_table()[O.payload(v, b, O.RCEIL)]
        assert 224.0 <= y <= 448.0


# ---------------------------------------------------------------------------
# dim0 cast: round-trip bound and known blocks
# ---------------------------------------------------------------------------
def _bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("mode", [O.RCEIL, O.FLOOR])
def test_dim0_round_trip_error_bound(mode):
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(64, 256, generator=g) * torch.exp2(torch.randint(-20, 20, (64, 1), generator=g).float())).to(torch.bfloat16)
    q, s = O.quant_dim0(_bf16_bits(x), mode)
    back = O.dequant(q, s)
    xv = x.double().numpy()
    step = np.repeat(np.ldexp(1.0, s.astype(np.int64) - 127 - 9), 32, axis=1)  # subnormal step
    # RCEIL keeps the block max <= 448 (rounding only, 3 mantissa bits: 2^-4);
    # FLOOR scales it into [256, 512) and clamps at 448 (up to 2^-3).
    rel = 2.0 ** -4 if mode == O.RCEIL else 2.0 ** -3
    assert np.all(np.abs(back - xv) <= np.abs(xv) * rel + step / 2)


def test_dim0_constant_block_known_answer():
    x = torch.ones(1, 32, dtype=torch.bfloat16)
    q, s = O.quant_dim0(_bf16_bits(x), O.RCEIL)
    assert s[0, 0] == 119 and np.all(q == 0x78)      # 1.0 * 2^8 = 256 -> 0x78
    x = torch.full((1, 32), 448.0, dtype=torch.bfloat16)
    q, s = O.quant_dim0(_bf16_bits(x), O.RCEIL)
    assert s[0, 0] == 127 and np.all(q == 0x7E)
    x = torch.zeros(1, 32, dtype=torch.bfloat16)
    q, s = O.quant_dim0(_bf16_bits(x), O.RCEIL)
    assert s[0, 0] == 0 and np.all(q == 0)


# ---------------------------------------------------------------------------
# dim1 cast: relation to dim0
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("mode", [O.RCEIL, O.FLOOR])
def test_dim1_equals_transposed_dim0_per_group(mode):
    g = torch.Generator().manual_seed(4)
    sizes = [5, 0, 64, 33, 1, 40]
    M = sum(sizes)
    x = torch.randn(M, 16, generator=g).to(torch.bfloat16)
    ends = np.cumsum(sizes).astype(np.int32)
    cap = (M + 31 * len(sizes) + 31) // 32 * 32
    qt, st, pad = O.quant_dim1(_bf16_bits(x), ends, cap, mode)
    b = 0
    p = 0
    for sz, e in zip(sizes, ends):
        padded = (sz + 31) // 32 * 32
        blk = torch.zeros(padded, 16, dtype=torch.bfloat16)
        blk[:sz] = x[b:e]
        q0, s0 = O.quant_dim0(_bf16_bits(blk.t().contiguous()), mode)
        assert np.array_equal(qt[:, p:p + padded], q0)
        assert np.array_equal(st[:, p // 32:(p + padded) // 32], s0)
        p += padded
        b = e
    assert list(pad) == list(np.cumsum([(s + 31) // 32 * 32 for s in sizes]))
    assert np.all(qt[:, p:] == 0)


# ---------------------------------------------------------------------------
# group ends: the running-maximum rule for malformed (decreasing / out of
# range) ends, stated independently with numpy
# ---------------------------------------------------------------------------
def _bounds_numpy(ends, rows):
    m = np.clip(np.maximum.accumulate(np.asarray(ends, dtype=np.int64)), 0, rows)
    return list(zip(np.r_[0, m[:-1]].tolist(), m.tolist()))


@pytest.mark.parametrize("seed", range(6))
def test_group_bounds_running_max_rule(seed):
    rng = np.random.default_rng(seed)
    rows = int(rng.integers(1, 500))
    ends = rng.integers(-50, rows + 80, int(rng.integers(1, 12)))
    b = O.group_bounds(ends, rows)
    assert b == _bounds_numpy(ends, rows)
    # disjoint, contiguous from row 0, sizes sum to at most rows
    assert b[0][0] == 0 and all(b[i][1] == b[i + 1][0] for i in range(len(b) - 1))
    assert all(t >= s for s, t in b) and sum(t - s for s, t in b) <= rows
    # well-formed cumulative ends are used as given
    ok = np.sort(rng.integers(0, rows + 1, 5))
    assert O.group_bounds(ok, rows) == list(zip(np.r_[0, ok[:-1]].tolist(), ok.tolist()))


@pytest.mark.parametrize("seed", range(4))
def test_rows_in_groups_is_the_union_of_the_group_ranges(seed):
    rng = np.random.default_rng(100 + seed)
    rows = int(rng.integers(1, 400))
    ends = rng.integers(-20, rows + 40, int(rng.integers(1, 10)))
    m = np.clip(np.maximum.accumulate(ends.astype(np.int64)), 0, rows)
    want = np.arange(rows) < m[-1]      # the groups tile [0, last running max)
    assert np.array_equal(O.rows_in_groups(ends, rows), want)


def test_gemm_comparison_checks_nan_rows_and_masks_only_what_it_is_told():
    # the comparison used by every GPU GEMM test: a reference row holding a
    # NaN is compared (the output must hold NaN at the same places), and rows
    # are skipped only through an explicit mask
    from tests._helpers import assert_close_to_oracle

    ref = np.arange(12, dtype=np.float64).reshape(4, 3) + 1.0
    ref[1, 2] = np.nan
    y = torch.from_numpy(ref.copy()).float()
    assert_close_to_oracle(y, ref)
    y_bad = y.clone()
    y_bad[1, 2] = 5.0
    with pytest.raises(AssertionError):
        assert_close_to_oracle(y_bad, ref)
    y_bad = y.clone()
    y_bad[3, 0] = float("nan")
    with pytest.raises(AssertionError):
        assert_close_to_oracle(y_bad, ref)
    y_off = y.clone()
    y_off[0] += 1.0
    with pytest.raises(AssertionError):
        assert_close_to_oracle(y_off, ref)
    assert_close_to_oracle(y_off, ref, rows=np.array([False, True, True, True]))
    assert_close_to_oracle(y_off, ref, rows=np.array([1, 2, 3]))


@pytest.mark.parametrize("ends", [[30, 10, 50], [80, 0, 80, 0], [-3, 20, 5, 200]])
def test_dim1_decreasing_ends_equal_their_running_max(ends):
    g = torch.Generator().manual_seed(7)
    M = 80
    x = _bf16_bits(torch.randn(M, 8, generator=g).to(torch.bfloat16))
    e = np.array(ends, dtype=np.int32)
    mono = np.clip(np.maximum.accumulate(e), 0, M).astype(np.int32)
    cap = (M + 31 * len(ends) + 31) // 32 * 32
    a = O.quant_dim1(x, e, cap)
    b = O.quant_dim1(x, mono, cap)
    for u, v in zip(a, b):
        assert np.array_equal(u, v)


# ---------------------------------------------------------------------------
# GEMM references
# ---------------------------------------------------------------------------
def _kat(name):
    return json.loads((GOLDEN / "scale_kats.json").read_text())[name]


def _ones_fp8(*shape):
    return np.full(shape, 0x38, dtype=np.uint8)  # e4m3 1.0


def test_kat_scale_byte_interpretation():
    k = _kat("scale_bypass")  # scale_correctness.py:181-251
    M, N, K, E = k["M"], k["N"], k["K"], k["E"]
    a_s = np.array(k["a_scale_row"], dtype=np.uint8)[None, :].repeat(M, 0)
    w_s = np.full((E, N, K // 32), 127, np.uint8)
    y = O.grouped_fwd(_ones_fp8(M, K), a_s, _ones_fp8(E, N, K), w_s, np.array(k["ends"]))
    assert np.all(y == k["expected"])


def test_kat_scale_application_order():
    k = _kat("application_order")  # scale_correctness.py:258-337
    M, N, K = k["M"], k["N"], k["K"]
    a_s = np.array(k["a_scale_row"], dtype=np.uint8)[None, :].repeat(M, 0)
    w_s = np.array(k["w_scale_row"], dtype=np.uint8)[None, None, :].repeat(N, 1)
    y = O.grouped_fwd(_ones_fp8(M, K), a_s, _ones_fp8(1, N, K), w_s, np.array(k["ends"]))
    assert np.all(y == k["expected"])


def test_kat_scale_layout_per_row():
    k = _kat("scale_layout")  # scale_correctness.py:344-401
    M, N, K = k["M"], k["N"], k["K"]
    a_s = np.full((M, K // 32), 127, np.uint8)
    a_s[:, 0] = np.minimum(127 + np.arange(M), 254)
    w_s = np.full((1, N, K // 32), 127, np.uint8)
    y = O.grouped_fwd(_ones_fp8(M, K), a_s, _ones_fp8(1, N, K), w_s, np.array(k["ends"]))
    expect = 32.0 * np.ldexp(1.0, a_s[:, 0].astype(int) - 127) + 32.0
    # exact while 32*2^m + 32 fits in 53 bits; beyond, each of the 32 unit terms
    # may round away (relative 32 * 2^-53)
    assert np.allclose(y, np.repeat(expect[:, None], N, 1), rtol=2.0 ** -47, atol=0.0)
    assert np.array_equal(y[:40], np.repeat(expect[:40, None], N, 1))


def test_kat_known_scales_against_torch_dequant():
    # scale_correctness.py:52-174: arange data, A scales alternating 2.0/1.0 per block.
    M, N, K, E = 64, 96, 128, 2
    # the reference's arange * 0.1 data, wrapped below 400 so it stays finite in e4m3
    a_vals = ((torch.arange(M * K, dtype=torch.float32) % 4000).reshape(M, K) * 0.1).to(torch.bfloat16)
    w_vals = ((torch.arange(E * N * K, dtype=torch.float32) % 4000).reshape(E, N, K) * 0.1).to(
        torch.bfloat16)
    a_s = np.full((M, K // 32), 127, np.uint8)
    a_s[:, ::2] = 128
    w_s = np.full((E, N, K // 32), 127, np.uint8)
    sa = torch.from_numpy(np.ldexp(1.0, a_s.astype(np.int64) - 127)).repeat_interleave(32, 1)
    sw = torch.from_numpy(np.ldexp(1.0, w_s.astype(np.int64) - 127)).repeat_interleave(32, 2)
    a_q = (a_vals.double() / sa).float().to(torch.float8_e4m3fn)
    w_q = (w_vals.double() / sw).float().to(torch.float8_e4m3fn)
    # independent reference: torch's float8 decode, float64 matmul per group
    ref = torch.empty(M, N, dtype=torch.float64)
    ref[:32] = (a_q[:32].double() * sa[:32]) @ (w_q[0].double() * sw[0]).T
    ref[32:] = (a_q[32:].double() * sa[32:]) @ (w_q[1].double() * sw[1]).T
    y = O.grouped_fwd(a_q.view(torch.uint8).numpy(), a_s, w_q.view(torch.uint8).numpy(), w_s,
                      np.array([32, 64]))
    assert np.array_equal(y, ref.numpy())


def test_grouped_fwd_brute_force_loops():
    rng = np.random.default_rng(5)
    M, N, K, E = 11, 5, 64, 4
    ends = np.array([3, 3, 9, 11])  # group 1 empty
    a_q = rng.integers(0, 0x7E, (M, K)).astype(np.uint8) | (rng.integers(0, 2, (M, K)) << 7).astype(np.uint8)
    w_q = rng.integers(0, 0x7E, (E, N, K)).astype(np.uint8)
    a_s = rng.integers(120, 134, (M, K // 32)).astype(np.uint8)
    w_s = rng.integers(120, 134, (E, N, K // 32)).astype(np.uint8)
    y = O.grouped_fwd(a_q, a_s, w_q, w_s, ends)
    tdec = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).double()
    dec = lambda c: float(tdec[int(c)])
    beg = 0
    for g, e in enumerate(ends):
        for m in range(beg, e):
            for n in range(N):
                acc = 0.0
                for k in range(K):
                    acc += (dec(a_q[m, k]) * 2.0 ** (int(a_s[m, k // 32]) - 127)
                            * dec(w_q[g, n, k]) * 2.0 ** (int(w_s[g, n, k // 32]) - 127))
                assert y[m, n] == pytest.approx(acc, rel=1e-12, abs=1e-300)
        beg = e


def test_scale_bump_doubles_output_exactly():
    rng = np.random.default_rng(6)
    M, N, K, E = 40, 24, 96, 2
    a_q = rng.integers(0, 0x7E, (M, K)).astype(np.uint8)
    w_q = rng.integers(0, 0x7E, (E, N, K)).astype(np.uint8)
    a_s = rng.integers(110, 140, (M, K // 32)).astype(np.uint8)
    w_s = rng.integers(110, 140, (E, N, K // 32)).astype(np.uint8)
    ends = np.array([17, 40])
    y = O.grouped_fwd(a_q, a_s, w_q, w_s, ends)
    y2 = O.grouped_fwd(a_q, a_s + 1, w_q, w_s, ends)
    assert np.array_equal(y2, 2.0 * y)


def test_wgrad_brute_force_loops():
    rng = np.random.default_rng(7)
    N, K, M = 3, 4, 96
    ends = np.array([32, 32, 96])  # group 1 empty
    go = rng.integers(0, 0x7E, (N, M)).astype(np.uint8)
    ia = rng.integers(0, 0x7E, (K, M)).astype(np.uint8)
    gs = rng.integers(120, 134, (N, M // 32)).astype(np.uint8)
    is_ = rng.integers(120, 134, (K, M // 32)).astype(np.uint8)
    dw = O.grouped_wgrad(go, gs, ia, is_, ends)
    dec = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    beg = 0
    for g, e in enumerate(ends):
        for n in range(N):
            for k in range(K):
                acc = sum(dec[go[n, t]] * 2.0 ** (int(gs[n, t // 32]) - 127) * dec[ia[k, t]]
                          * 2.0 ** (int(is_[k, t // 32]) - 127) for t in range(beg, e))
                assert dw[g, n, k] == pytest.approx(acc, rel=1e-12, abs=0.0)
        beg = e
    assert np.all(dw[1] == 0)


# ---------------------------------------------------------------------------
# golden fixture (config 1)
# ---------------------------------------------------------------------------
def test_c1_golden_fixture():
    import hashlib
    import sys

    sys.path.insert(0, str(Path(__file__).resolve().parent.parent / "mxfp8-grouped-gemm_amd"))
    from mxfp8gg import workloads

    fx = json.loads((GOLDEN / "c1_golden.json").read_text())
    x, w, sizes = workloads.c1("cpu")
    xq, xs = O.quant_dim0(_bf16_bits(x), O.RCEIL)
    wq, ws = O.quant_dim0(_bf16_bits(w.reshape(-1, 256)), O.RCEIL)
    h = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    assert h(_bf16_bits(x)) == fx["x_sha256"]
    assert h(xq) == fx["xq_sha256"] and h(xs) == fx["xs_sha256"]
    assert h(wq) == fx["wq_sha256"] and h(ws) == fx["ws_sha256"]
    y = O.grouped_fwd(xq, xs, wq.reshape(4, 512, 256), ws.reshape(4, 512, 8),
                      workloads.ends_of(sizes))
    probe = np.array(fx["y_probe"])
    idx = np.array(fx["y_probe_index"])
    assert np.allclose(y[idx[:, 0], idx[:, 1]], probe, rtol=0, atol=1e-9)


# ---------------------------------------------------------------------------
# SwiGLU activation (expert FFN): pinned against torch's CPU bf16 eager ops
# and autograd (an independent implementation with its own exp), and against
# the float64 closed form of the derivative.
# ---------------------------------------------------------------------------
def _bf16_inputs(n, seed, scale=3.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(n, generator=g) * scale).to(torch.bfloat16)
    return x, x.view(torch.int16).numpy().view(np.uint16)


def _ulp_diff(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    sa = np.where(a & 0x8000, -(a & 0x7FFF), a)
    sb = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(sa - sb)


def test_swiglu_fwd_matches_torch_cpu_bf16():
    gt, gb = _bf16_inputs(200000, 1)
    ut, ub = _bf16_inputs(200000, 2, 1.0)
    ref = (torch.nn.functional.silu(gt) * ut).view(torch.int16).numpy().view(np.uint16)
    got = O.swiglu_fwd(gb, ub)
    diff = _ulp_diff(got, ref)
    assert diff.max() <= 1
    assert (diff > 0).mean() < 1e-3  # exp implementations may differ in the last fp32 bit


def test_swiglu_bwd_matches_torch_cpu_autograd():
    gt, gb = _bf16_inputs(100000, 3)
    ut, ub = _bf16_inputs(100000, 4, 1.0)
    dt, db = _bf16_inputs(100000, 5, 0.01)
    g_ = gt.clone().requires_grad_(True)
    u_ = ut.clone().requires_grad_(True)
    a = torch.nn.functional.silu(g_) * u_
    a.backward(dt)
    a_o, dg_o, du_o = O.swiglu_bwd(gb, ub, db)
    for got, ref in ((a_o, a), (dg_o, g_.grad), (du_o, u_.grad)):
        r = ref.detach().view(torch.int16).numpy().view(np.uint16)
        diff = _ulp_diff(got, r)
        assert diff.max() <= 1
        assert (diff > 0).mean() < 1e-3


def test_swiglu_derivative_closed_form_float64():
    # d/dg [g * sigmoid(g) * u] = u * sig * (1 + g * (1 - sig)); d/du = silu(g)
    gt, gb = _bf16_inputs(50000, 6)
    ut, ub = _bf16_inputs(50000, 7, 1.0)
    dt, db = _bf16_inputs(50000, 8, 0.01)
    g = gt.double().numpy()
    u = ut.double().numpy()
    d = dt.double().numpy()
    sig = 1.0 / (1.0 + np.exp(-g))
    dg_ref = d * u * sig * (1.0 + g * (1.0 - sig))
    du_ref = d * g * sig
    a_ref = g * sig * u
    a_o, dg_o, du_o = (O.bits_to_f32(x).astype(np.float64) for x in O.swiglu_bwd(gb, ub, db))
    # three bf16 roundings in a chain: within 4 bf16 half-ulps of the exact value
    for got, ref in ((a_o, a_ref), (dg_o, dg_ref), (du_o, du_ref)):
        assert np.all(np.abs(got - ref) <= 2.0 ** -7 * np.abs(ref) + 1e-30)
    # the forward of the backward oracle is the forward oracle
    assert np.array_equal(O.swiglu_bwd(gb, ub, db)[0], O.swiglu_fwd(gb, ub))


def test_swiglu_special_points():
    g = np.array([0.0, 20.0, -20.0, np.inf, -np.inf, np.nan], np.float32)
    u = np.ones_like(g)
    d = np.ones_like(g)
    gb = O.f32_to_bits(g)
    a, dg, du = (O.bits_to_f32(x) for x in O.swiglu_bwd(gb, O.f32_to_bits(u), O.f32_to_bits(d)))
    assert a[0] == 0 and du[0] == 0 and dg[0] == 0.5          # silu(0) = 0, silu'(0) = 1/2
    assert a[1] == 20.0 and dg[1] == 1.0                       # sig(20) rounds to 1 in bf16 math
    assert abs(a[2]) < 1e-7 and abs(dg[2]) < 1e-6
    assert a[3] == np.inf and np.isnan(a[4])                   # -inf / (1 + inf) = NaN
    assert np.isnan(a[5]) and np.isnan(dg[5]) and np.isnan(du[5])


# ---------------------------------------------------------------------------
# Token routing (dispatch plan, gather, combine)
# ---------------------------------------------------------------------------
def test_route_plan_known_answer():
    # slots 0..5 go to experts 2,0,0,1,2,2; groups padded to 4 rows
    perm, src, ends, counts = O.route_plan(np.array([[2, 0], [0, 1], [2, 2]]), 3, 4, 16)
    assert perm.tolist() == [8, 0, 1, 4, 9, 10]
    assert src.tolist() == [1, 2, -1, -1, 3, -1, -1, -1, 0, 4, 5, -1, -1, -1, -1, -1]
    assert ends.tolist() == [4, 8, 12] and counts.tolist() == [2, 1, 3]


@pytest.mark.parametrize("T,K,E,pad,seed", [(50, 1, 4, 1, 0), (300, 8, 32, 1, 1), (97, 3, 7, 32, 2),
                                            (64, 8, 256, 128, 3), (5, 2, 1, 32, 4)])
def test_route_plan_is_torch_stable_argsort(T, K, E, pad, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, E, (T, K), generator=g)
    perm, src, ends, counts = O.route_plan(idx.numpy(), E, pad, T * K + E * (pad - 1))
    order = torch.argsort(idx.reshape(-1), stable=True).numpy()   # torchtitan's dispatch order
    assert np.array_equal(src[src >= 0], order)
    assert np.array_equal(perm[src[src >= 0]], np.flatnonzero(src >= 0))
    assert np.array_equal(counts, torch.bincount(idx.reshape(-1), minlength=E).numpy())
    padded = -(-counts // pad) * pad
    assert np.array_equal(ends, np.cumsum(padded))
    for e in range(E):   # each group: its slots first, then empty rows
        lo = ends[e] - padded[e]
        assert np.all(src[lo:lo + counts[e]] >= 0) and np.all(src[lo + counts[e]:ends[e]] == -1)
    assert np.all(src[ends[-1]:] == -1)


def test_route_plan_drops_out_of_range_ids():
    idx = np.array([[0, 5], [-1, 1], [1, 0]])
    perm, src, ends, counts = O.route_plan(idx, 2, 1, 6)
    assert perm.tolist() == [0, -1, -1, 2, 3, 1]
    assert counts.tolist() == [2, 2] and ends.tolist() == [2, 4]
    assert src.tolist() == [0, 5, 3, 4, -1, -1]


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_gather_and_combine_match_torch_index_ops():
    g = torch.Generator().manual_seed(5)
    T, K, E, H = 40, 4, 6, 24
    idx = torch.randint(0, E, (T, K), generator=g)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    sc = torch.rand(T, K, generator=g)
    perm, src, ends, _ = O.route_plan(idx.numpy(), E, 1, T * K)
    order = torch.argsort(idx.reshape(-1), stable=True)
    # gather: the dispatcher's routed input x[sorted // topk], and its scaled form
    assert np.array_equal(O.gather_rows(_bf16_bits(x), src, K), _bf16_bits(x[order // K]))
    scaled = (x[order // K].float() * sc.reshape(-1)[order][:, None]).to(torch.bfloat16)
    assert np.array_equal(O.gather_rows(_bf16_bits(x), src, K, sc.numpy()), _bf16_bits(scaled))
    # combine with topk = 1 puts every routed row back in place
    perm1, src1, _, _ = O.route_plan(idx[:, :1].numpy(), E, 1, T)
    y1 = O.gather_rows(_bf16_bits(x), src1, 1)
    assert np.array_equal(O.combine(y1, perm1, 1), _bf16_bits(x))
    # combine: the dispatcher's scaled scatter-add, summed exactly (float64)
    y = torch.randn(T * K, H, generator=g).to(torch.bfloat16)
    terms = (y[torch.from_numpy(perm).long()].float() * sc.reshape(-1)[:, None]).to(torch.bfloat16)
    exact = torch.zeros(T, H, dtype=torch.float64).index_add_(
        0, torch.arange(T).repeat_interleave(K), terms.double())
    got = O.bits_to_f32(O.combine(_bf16_bits(y), perm, K, sc.numpy())).astype(np.float64)
    ref = exact.to(torch.bfloat16).float().numpy().astype(np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
    assert np.all(np.abs(got - ref) <= ulp)                # at most one bf16 ulp (fp32 sum order)
    assert np.mean(got != ref) < 0.01


def test_combine_score_grad_matches_torch_autograd():
    g = torch.Generator().manual_seed(6)
    T, K, E, H = 16, 2, 3, 32
    idx = torch.randint(0, E, (T, K), generator=g)
    perm, _, _, _ = O.route_plan(idx.numpy(), E, 1, T * K)
    y = torch.randn(T * K, H, generator=g).to(torch.bfloat16)
    d = torch.randn(T, H, generator=g).to(torch.bfloat16)
    sc = torch.rand(T, K, generator=g, dtype=torch.float64).requires_grad_(True)
    # the combine as torch ops (rounding steps are identity for autograd)
    terms = y[torch.from_numpy(perm).long()].double().reshape(T, K, H) * sc[:, :, None]
    out = terms.sum(1)
    out.backward(d.double())
    got = O.combine_score_grad(_bf16_bits(d), _bf16_bits(y), perm, K)
    assert np.allclose(got, sc.grad.numpy(), rtol=1e-12, atol=1e-12)
