"""GPU parity of the gate+up GEMM fused with SwiGLU and the MXFP8 cast
(mxgg_grouped_fwd_swiglu_quant, and mxgg_grouped_fwd_swiglu_quant_keep_h,
which also writes the bf16 projection h for the training backward) through
the C ABI.

The fused kernels must give the same bytes as the unfused path they replace
-- the grouped GEMM's bf16 output h followed by the standalone SwiGLU cast,
each pinned against the oracle by tests/test_gpu_gemm.py and
tests/test_gpu_swiglu.py -- on every row inside the groups, for both scale
modes, both scale layouts, scaled and unscaled operands, ragged and empty
groups, and at C5's full shape; the kept h equals the GEMM's bf16 output bit
for bit.  An independent check against the oracle's float64 GEMM and float64
SiLU * up pins the pairing of gate and up columns."""
import numpy as np
import pytest
import torch

import mxfp8gg
from mxfp8gg import _lib, ops, workloads
from oracle import oracle as O
from tests._helpers import u8

pytestmark = pytest.mark.gpu


def _operands(gpu, sizes, F, K, seed, mode="rceil"):
    E, M = len(sizes), int(np.sum(sizes))
    g = torch.Generator(device=gpu).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=gpu).to(torch.bfloat16)
    w = (torch.randn(E, 2 * F, K, generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    xq, xs = mxfp8gg.to_mxfp8_dim0(x, mode)
    wq, ws = mxfp8gg.to_mxfp8_dim0(w, mode)
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    return xq, xs, wq, ws, offs


def _inside(sizes, gpu):
    ends = workloads.ends_of(sizes)
    mask = np.zeros(int(np.sum(sizes)), bool)
    for b, t in O.group_bounds(ends, mask.size):
        mask[b:t] = True
    return torch.from_numpy(mask).to(gpu)


@pytest.mark.parametrize("sizes,F,K", [
    ([64, 0, 300, 33], 128, 256),     # empty expert, starts off multiples of 4 and 32
    ([7, 250, 1, 0], 256, 384),       # tiny groups, K % 128 = 0 with 3 stages
    ([513], 384, 128),                # one expert, M tail, three feature tiles
])
@pytest.mark.parametrize("scaled", [True, False])
@pytest.mark.parametrize("mode", ["rceil", "floor"])
def test_fused_gate_up_equals_unfused(gpu, sizes, F, K, scaled, mode):
    xq, xs, wq, ws, offs = _operands(gpu, sizes, F, K, 131, mode)
    if not scaled:
        xs = ws = None
    q, s = ops.grouped_mm_swiglu_quant(xq, wq, offs, xs, ws, mode)
    h = ops.grouped_mm(xq, wq, offs, xs, ws, split_tail=False)  # the fused kernel never splits
    rq, rs = ops.swiglu_quant(h, mode)
    ins = _inside(sizes, gpu)
    assert q.shape == rq.shape and s.shape == rs.shape
    assert torch.equal(q.view(torch.uint8)[ins], rq.view(torch.uint8)[ins])
    assert torch.equal(s[ins], rs[ins])
    # the training variant: the same cast plus h itself
    qk, sk, hk = ops.grouped_mm_swiglu_quant(xq, wq, offs, xs, ws, mode, return_h=True)
    assert hk.shape == h.shape and hk.dtype == torch.bfloat16
    assert torch.equal(hk.view(torch.int16)[ins], h.view(torch.int16)[ins])
    assert torch.equal(qk.view(torch.uint8)[ins], rq.view(torch.uint8)[ins])
    assert torch.equal(sk[ins], rs[ins])


def test_fused_keep_h_strides_and_rows_past_the_end(gpu):
    # through the C ABI: h with a padded row stride, rows past the last group
    # end and the padding columns must keep their fill bytes
    sizes, F, K = [70, 0, 121], 128, 256
    xq, xs, wq, ws, offs = _operands(gpu, sizes, F, K, 135)
    tail = 37
    xq = torch.cat([xq, xq[:tail]])
    xs = torch.cat([xs.contiguous(), xs[:tail].contiguous()])
    M, E = xq.shape[0], wq.shape[0]
    sa, ldas = ops._scales_2d(xs, M, K // 32, "xs")
    sw, wsg, ldws = ops._scales_3d(ws, E, 2 * F, K // 32, "ws")
    ldh, ldq = 2 * F + 24, F + 40
    h = torch.full((M, ldh), 0x7FC1, dtype=torch.int16, device=gpu)
    q = torch.full((M, ldq), 0xAB, dtype=torch.uint8, device=gpu)
    s = torch.full((F // 32, (M + 15) // 16 * 16), 0xCD, dtype=torch.uint8, device=gpu)
    lib = _lib.load()
    st = lib.mxgg_grouped_fwd_swiglu_quant_keep_h(
        xq.data_ptr(), K, sa.data_ptr(), ldas, wq.data_ptr(), 2 * F * K, K, sw.data_ptr(), wsg,
        ldws, offs.data_ptr(), E, M, F, K, h.data_ptr(), ldh, q.data_ptr(), ldq, s.data_ptr(),
        s.stride(0), _lib.SCALES_BLOCK_MAJOR, _lib.SCALE_RCEIL,
        torch.cuda.current_stream(gpu).cuda_stream)
    assert st == 0, lib.mxgg_last_error()
    torch.cuda.synchronize(gpu)
    inside = int(np.sum(sizes))
    h_ref = ops.grouped_mm(xq[:inside], wq, offs, xs[:inside], ws, split_tail=False)
    rq, rs = ops.swiglu_quant(h_ref)
    assert torch.equal(h[:inside, :2 * F], h_ref.view(torch.int16))
    assert torch.equal(q[:inside, :F], rq.view(torch.uint8))
    assert torch.equal(s[:, :inside], rs.t())
    assert bool((h[inside:] == 0x7FC1).all()) and bool((h[:, 2 * F:] == 0x7FC1).all())
    assert bool((q[inside:] == 0xAB).all()) and bool((q[:, F:] == 0xAB).all())
    assert bool((s[:, inside:M] == 0xCD).all())


def test_fused_row_major_scales_through_the_c_abi(gpu):
    sizes, F, K = [100, 0, 156], 256, 256
    xq, xs, wq, ws, offs = _operands(gpu, sizes, F, K, 132)
    q_bm, s_bm = ops.grouped_mm_swiglu_quant(xq, wq, offs, xs, ws)
    M, E = xq.shape[0], wq.shape[0]
    sa, ldas = ops._scales_2d(xs, M, K // 32, "xs")
    sw, wsg, ldws = ops._scales_3d(ws, E, 2 * F, K // 32, "ws")
    q = torch.zeros((M, F), dtype=torch.uint8, device=gpu)
    s = torch.zeros((M, F // 32), dtype=torch.uint8, device=gpu)
    lib = _lib.load()
    st = lib.mxgg_grouped_fwd_swiglu_quant(
        xq.data_ptr(), K, sa.data_ptr(), ldas, wq.data_ptr(), 2 * F * K, K, sw.data_ptr(), wsg,
        ldws, offs.data_ptr(), E, M, F, K, q.data_ptr(), F, s.data_ptr(), F // 32,
        _lib.SCALES_ROW_MAJOR, _lib.SCALE_RCEIL, torch.cuda.current_stream(gpu).cuda_stream)
    assert st == 0, lib.mxgg_last_error()
    assert torch.equal(q, q_bm.view(torch.uint8)) and torch.equal(s, s_bm.contiguous())


def test_fused_pairs_gate_with_its_up_column(gpu):
    # independent of the unfused path: dequantised a against SiLU(g) * u of the
    # oracle's float64 gate+up GEMM (a swapped or shifted column pairing fails)
    sizes, F, K = [96, 160], 256, 192
    xq, xs, wq, ws, offs = _operands(gpu, sizes, F, K, 133)
    q, s = ops.grouped_mm_swiglu_quant(xq, wq, offs, xs, ws)
    h = O.grouped_fwd(u8(xq), u8(xs), u8(wq), u8(ws), workloads.ends_of(sizes))
    g, u = h[:, :F], h[:, F:]
    a_ref = g / (1.0 + np.exp(-g)) * u
    a_got = O.dequant(u8(q), u8(s))
    err = np.abs(a_got - a_ref)
    # e4m3 payload (3 mantissa bits) after two bf16 roundings
    assert np.all(err <= 2.0 ** -3 * np.abs(a_ref) + 2.0 ** -8 * np.abs(a_ref).max())
    assert err.max() / np.abs(a_ref).max() < 0.07


def test_fused_c5_shape(gpu):
    sizes = workloads.c5_sizes()
    H, F = 7168, 2048
    print(f"C5 gate+up fused: {int(sizes.sum())} tokens", flush=True)
    xq, xs, wq, ws, offs = _operands(gpu, sizes, F, H, 0)
    q, s = ops.grouped_mm_swiglu_quant(xq, wq, offs, xs, ws)
    h = ops.grouped_mm(xq, wq, offs, xs, ws, split_tail=False)
    rq, rs = ops.swiglu_quant(h)
    assert torch.equal(q.view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(s, rs)
    del q, s
    qk, sk, hk = ops.grouped_mm_swiglu_quant(xq, wq, offs, xs, ws, return_h=True)
    assert torch.equal(hk.view(torch.int16), h.view(torch.int16))
    assert torch.equal(qk.view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(sk, rs)


def test_forward_only_layers_equal_the_training_forward(gpu):
    sizes = [64, 0, 200, 33]
    E, H, F = 4, 256, 128
    g = torch.Generator(device=gpu).manual_seed(134)
    M = sum(sizes)
    x = torch.randn(M, H, generator=g, device=gpu).to(torch.bfloat16)
    wgu = (torch.randn(E, 2 * F, H, generator=g, device=gpu) * 0.06).to(torch.bfloat16)
    wd = (torch.randn(E, H, F, generator=g, device=gpu) * 0.06).to(torch.bfloat16)
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    with torch.no_grad():
        y0 = mxfp8gg.moe_ffn(x, wgu, wd, offs)               # fused gate+up path
    y1 = mxfp8gg.moe_ffn(x, wgu.requires_grad_(True), wd, offs)  # training path (bf16 h)
    assert torch.equal(y0, y1.detach())
    idx = torch.randint(0, E, (48, 2), generator=g, device=gpu, dtype=torch.int32)
    sc = torch.rand(48, 2, generator=g, device=gpu)
    xr = torch.randn(48, H, generator=g, device=gpu).to(torch.bfloat16)
    with torch.no_grad():
        r0 = mxfp8gg.moe_routed_ffn(xr, idx, sc, wgu, wd)
    r1 = mxfp8gg.moe_routed_ffn(xr, idx, sc, wgu, wd)        # wgu requires grad
    assert torch.equal(r0, r1.detach())
