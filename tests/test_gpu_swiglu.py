"""GPU parity of the fused SwiGLU kernels (expert FFN activation + its casts)
through the C ABI.

The activation is floating point: the kernel's bf16 results are compared with
the CPU oracle (float32 math, bf16 rounding after every op) to at most one
bf16 ulp in a small fraction of elements (numpy's and the GPU's exp differ in
the last fp32 bit), and with torch's own GPU eager ops, which they match bit
for bit (at most one value in a million may differ by one ulp).  Every cast the kernels
write is then checked bit for bit against the oracle's cast of the kernel's
own bf16 values, so the quantisation parity is exact."""
import numpy as np
import pytest
import torch

import mxfp8gg
from mxfp8gg import workloads
from oracle import oracle as O
from tests._helpers import bits, u8

pytestmark = pytest.mark.gpu

MAX_ULP_FRACTION = 1e-3     # vs the numpy oracle
TORCH_ULP_FRACTION = 1e-6   # vs torch's GPU eager ops


def _ulp_diff(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    sa = np.where(a & 0x8000, -(a & 0x7FFF), a)
    sb = np.where(b & 0x8000, -(b & 0x7FFF), b)
    d = np.abs(sa - sb)
    nan_a = ((a & 0x7F80) == 0x7F80) & ((a & 0x7F) != 0)
    nan_b = ((b & 0x7F80) == 0x7F80) & ((b & 0x7F) != 0)
    d[nan_a & nan_b] = 0  # NaN payload bits are not compared
    d[nan_a ^ nan_b] = 1 << 16
    return d


def _assert_bf16_close(got_bits, ref_bits, what, frac=MAX_ULP_FRACTION):
    assert got_bits.shape == ref_bits.shape
    if got_bits.size == 0:
        return
    d = _ulp_diff(got_bits, ref_bits)
    assert d.max() <= 1, f"{what}: {int(d.max())} ulp at {np.unravel_index(d.argmax(), d.shape)}"
    assert (d > 0).mean() <= frac, f"{what}: {(d > 0).mean():.2e} of values differ"


def _h(gpu, M, F, seed, specials=False):
    g = torch.Generator(device=gpu).manual_seed(seed)
    h = torch.randn(M, 2 * F, generator=g, device=gpu) * 2.5
    h[:, F:] *= 0.4
    if M > 3:
        h[1] = 0.0                         # an all-zero row: zero payload, byte 0
        h[2, :F] = 30.0                    # saturated sigmoid
    if specials and M > 8:
        h[5, 3] = float("inf")
        h[6, F + 7] = float("-inf")
        h[7, 40] = float("nan")
    if specials and M > 10:
        # the kernels' range-test-free math takes rows whose gates all lie in
        # |g| <= 87: both edges of that domain; gates past it where
        # 1 + exp(-g) >= 2^126 has a reciprocal below the normal range
        # (-88.7 < g < -87.3); gates where exp(-g) overflows (g < -88.7) or
        # underflows to a denormal or zero (g > 87)
        h[8, :6] = torch.tensor([87.0, -87.0, 87.5, -87.5, 88.0, -88.0])
        h[9, :6] = torch.tensor([88.5, -88.5, 100.0, -100.0, 104.0, -104.0])
        h[10, 1::7] = -87.0
    return h.to(torch.bfloat16)


@pytest.mark.parametrize("mode_name,mode", [("rceil", O.RCEIL), ("floor", O.FLOOR)])
@pytest.mark.parametrize("M,F", [(1, 32), (37, 96), (300, 256)])
def test_swiglu_quant_dim0(gpu, mode_name, mode, M, F):
    h = _h(gpu, M, F, 11, specials=True)
    q, s, a = mxfp8gg.swiglu_quant(h, mode_name, return_bf16=True)
    hb = bits(h)
    a_ref = O.swiglu_fwd(hb[:, :F], hb[:, F:])
    _assert_bf16_close(bits(a), a_ref, "a vs oracle")
    torch_a = torch.nn.functional.silu(h[:, :F]) * h[:, F:]
    _assert_bf16_close(bits(a), bits(torch_a), "a vs torch eager", TORCH_ULP_FRACTION)
    rq, rs = O.quant_dim0(bits(a), mode)
    assert np.array_equal(u8(q), rq)
    assert np.array_equal(u8(s), rs)
    # without the bf16 copy the cast is the same
    q2, s2 = mxfp8gg.swiglu_quant(h, mode_name)
    assert torch.equal(q2.view(torch.uint8), q.view(torch.uint8))
    assert torch.equal(s2.contiguous(), s.contiguous())


def _bwd_inputs(gpu, sizes, F, seed, specials=False):
    M = int(sum(sizes))
    h = _h(gpu, M, F, seed, specials)
    g = torch.Generator(device=gpu).manual_seed(seed + 1)
    da = (torch.randn(M, F, generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(gpu) if sizes is not None else None
    return h, da, offs


@pytest.mark.parametrize("mode_name,mode", [("rceil", O.RCEIL), ("floor", O.FLOOR)])
@pytest.mark.parametrize("sizes,F", [([40, 0, 77, 33], 64), ([256], 96), ([5, 0, 0, 300, 17], 32),
                                     ([0, 0], 64)])
def test_swiglu_backward_quant(gpu, mode_name, mode, sizes, F):
    h, da, offs = _bwd_inputs(gpu, sizes, F, 21, specials=True)
    M = h.shape[0]
    out = mxfp8gg.swiglu_backward_quant(h, da, offs, mode_name, return_bf16=True)
    hb = bits(h)
    ends = workloads.ends_of(sizes)
    cap = mxfp8gg.padded_token_capacity(M, len(sizes))
    a_ref, dg_ref, du_ref = O.swiglu_bwd(hb[:, :F], hb[:, F:], bits(da))
    dh = bits(out["dh"])
    _assert_bf16_close(dh[:, :F], dg_ref, "d_gate vs oracle")
    _assert_bf16_close(dh[:, F:], du_ref, "d_up vs oracle")
    # torch's own eager autograd on the GPU
    gt = h[:, :F].clone().requires_grad_(True)
    ut = h[:, F:].clone().requires_grad_(True)
    (torch.nn.functional.silu(gt) * ut).backward(da)
    _assert_bf16_close(dh[:, :F], bits(gt.grad), "d_gate vs torch autograd", TORCH_ULP_FRACTION)
    _assert_bf16_close(dh[:, F:], bits(ut.grad), "d_up vs torch autograd", TORCH_ULP_FRACTION)
    # every cast is bit-exact against the oracle cast of the kernel's own values
    rq, rs = O.quant_dim0(dh, mode)
    assert np.array_equal(u8(out["dh_q"]), rq)
    assert np.array_equal(u8(out["dh_s"]), rs)
    rqt, rst, rpad = O.quant_dim1(dh, ends, cap, mode)
    assert np.array_equal(u8(out["dh_qt"]), rqt)
    assert np.array_equal(u8(out["dh_st"]), rst)
    assert np.array_equal(out["offs_pad"].cpu().numpy(), rpad)
    # a: the backward kernel recomputes exactly what the forward kernel writes
    _, _, a_fwd = mxfp8gg.swiglu_quant(h, mode_name, return_bf16=True)
    aqt, ast, _ = O.quant_dim1(bits(a_fwd), ends, cap, mode)
    assert np.array_equal(u8(out["a_qt"]), aqt)
    assert np.array_equal(u8(out["a_st"]), ast)


def test_swiglu_backward_single_group_and_no_bf16(gpu):
    h, da, _ = _bwd_inputs(gpu, [200], 64, 31)
    full = mxfp8gg.swiglu_backward_quant(h, da, None, return_bf16=True)
    lean = mxfp8gg.swiglu_backward_quant(h, da, None)
    for k in ("dh_q", "dh_qt", "a_qt"):
        assert torch.equal(full[k].view(torch.uint8), lean[k].view(torch.uint8))
    for k in ("dh_s", "dh_st", "a_st"):
        assert torch.equal(full[k].contiguous(), lean[k].contiguous())
    cap = mxfp8gg.padded_token_capacity(200, None)
    rqt, rst, _ = O.quant_dim1(bits(full["dh"]), None, cap)
    assert np.array_equal(u8(full["dh_qt"]), rqt)
    assert np.array_equal(u8(full["dh_st"]), rst)


def test_swiglu_backward_c5_shape_sampled(gpu):
    # DSv3 expert FFN: 131072 routed tokens, Zipf(1.0) over 32 experts, F = 2048.
    sizes = workloads.c5_sizes()
    F = 2048
    h, da, offs = _bwd_inputs(gpu, sizes, F, 41)
    out = mxfp8gg.swiglu_backward_quant(h, da, offs, return_bf16=True)
    rows = np.sort(np.random.default_rng(42).choice(h.shape[0], 64, replace=False))
    hb = bits(h[torch.from_numpy(rows).to(gpu)])
    _, dg_ref, du_ref = O.swiglu_bwd(hb[:, :F], hb[:, F:], bits(da[torch.from_numpy(rows).to(gpu)]))
    dh = bits(out["dh"][torch.from_numpy(rows).to(gpu)])
    _assert_bf16_close(dh[:, :F], dg_ref, "d_gate vs oracle")
    _assert_bf16_close(dh[:, F:], du_ref, "d_up vs oracle")
    rq, rs = O.quant_dim0(dh, O.RCEIL)
    assert np.array_equal(u8(out["dh_q"][torch.from_numpy(rows).to(gpu)]), rq)
    assert np.array_equal(u8(out["dh_s"][torch.from_numpy(rows).to(gpu)]), rs)
    # token-axis cast: the same bytes as the standalone cast of the bf16 dh
    qt, st, pad = mxfp8gg.to_mxfp8_dim1(out["dh"], offs)
    assert torch.equal(qt.view(torch.uint8), out["dh_qt"].view(torch.uint8))
    assert torch.equal(st.contiguous(), out["dh_st"].contiguous())
    assert torch.equal(pad, out["offs_pad"])
