"""GPU parity of the bf16 -> MXFP8 casts against the CPU oracle: bit-exact
payload and E8M0 bytes, both scale modes, both e4m3 encoders (hardware
v_cvt_pk_fp8_f32 and the bit-level software encoder)."""
import numpy as np
import pytest
import torch

import mxfp8gg
from mxfp8gg import _lib, ops, workloads
from oracle import oracle as O
from tests._helpers import bits, from_bits, u8

pytestmark = pytest.mark.gpu

MODES = [("rceil", O.RCEIL), ("floor", O.FLOOR)]
ENCODERS = [0, _lib.CVT_SOFTWARE]


def _dim0(x, mode_code):
    return ops.to_mxfp8_dim0(x, mode_code)


@pytest.mark.parametrize("name,mode", MODES)
@pytest.mark.parametrize("enc", ENCODERS)
def test_dim0_every_bf16_pattern(gpu, name, mode, enc):
    # all 65536 bit patterns (incl. NaN, Inf, subnormals, -0), in order and shuffled
    pats = np.arange(65536, dtype=np.uint16)
    rng = np.random.default_rng(11)
    x = np.concatenate([pats, rng.permutation(pats), rng.permutation(pats)]).reshape(-1, 256)
    q, s = _dim0(from_bits(x, gpu), mode | enc)
    rq, rs = O.quant_dim0(x, mode)
    assert np.array_equal(u8(s), rs)
    assert np.array_equal(u8(q), rq)


@pytest.mark.parametrize("name,mode", MODES)
def test_dim0_random_wide_dynamic_range(gpu, name, mode):
    g = torch.Generator(device=gpu).manual_seed(12)
    x = torch.randn(512, 1024, generator=g, device=gpu)
    x = x * torch.exp2(torch.randint(-60, 60, (512, 32), generator=g, device=gpu).float()
                       ).repeat_interleave(32, 1)
    x = x.to(torch.bfloat16)
    q, s = _dim0(x, mode)
    rq, rs = O.quant_dim0(bits(x), mode)
    assert np.array_equal(u8(s), rs) and np.array_equal(u8(q), rq)


@pytest.mark.parametrize("name,mode", MODES)
def test_dim0_row_major_scale_layout(gpu, name, mode):
    # the C ABI's ROW_MAJOR scale output (the reference's [M, K//32] layout)
    g = torch.Generator(device=gpu).manual_seed(17)
    x = (torch.randn(96, 512, generator=g, device=gpu) * 7).to(torch.bfloat16)
    q = torch.empty((96, 512), dtype=torch.float8_e4m3fn, device=gpu)
    s = torch.empty((96, 16), dtype=torch.uint8, device=gpu)
    lib = _lib.load()
    _lib.check(lib.mxgg_quant_dim0(x.data_ptr(), 96, 512, 512, q.data_ptr(), 512, s.data_ptr(), 16,
                                   _lib.SCALES_ROW_MAJOR, mode,
                                   torch.cuda.current_stream().cuda_stream), "dim0")
    rq, rs = O.quant_dim0(bits(x), mode)
    assert np.array_equal(u8(q), rq) and np.array_equal(u8(s), rs)
    q2, s2 = ops.to_mxfp8_dim0(x, mode)
    assert s2.stride() == (1, 96) and torch.equal(s2.contiguous(), s)


def test_dim0_strided_rows_and_3d(gpu):
    g = torch.Generator(device=gpu).manual_seed(13)
    base = torch.randn(64, 384, generator=g, device=gpu).to(torch.bfloat16)
    x = base[:, :256]  # ldx = 384 > cols
    q, s = ops.to_mxfp8_dim0(x)
    rq, rs = O.quant_dim0(bits(x), O.RCEIL)
    assert np.array_equal(u8(q), rq) and np.array_equal(u8(s), rs)
    w = torch.randn(3, 40, 96, generator=g, device=gpu).to(torch.bfloat16)
    q3, s3 = ops.to_mxfp8_dim0(w)
    assert q3.shape == (3, 40, 96) and s3.shape == (3, 40, 3)
    rq, rs = O.quant_dim0(bits(w.reshape(-1, 96)), O.RCEIL)
    assert np.array_equal(u8(q3).reshape(-1, 96), rq)
    assert np.array_equal(u8(s3).reshape(-1, 3), rs)


def test_dim0_c2_activation_sampled_rows(gpu):
    x, _, _ = workloads.c2(gpu)
    q, s = ops.to_mxfp8_dim0(x)
    rows = np.random.default_rng(14).choice(x.shape[0], 96, replace=False)
    rows.sort()
    rq, rs = O.quant_dim0(bits(x[torch.from_numpy(rows).to(gpu)]), O.RCEIL)
    idx = torch.from_numpy(rows).to(gpu)
    assert np.array_equal(u8(q[idx]), rq) and np.array_equal(u8(s[idx]), rs)
    del x, q, s


@pytest.mark.parametrize("name,mode", MODES)
@pytest.mark.parametrize("enc", ENCODERS)
@pytest.mark.parametrize("sizes", [[5, 0, 64, 33, 1, 40, 0], [128, 128], [300], [0, 0, 7]])
def test_dim1_grouped_matches_oracle(gpu, name, mode, enc, sizes):
    g = torch.Generator(device=gpu).manual_seed(15)
    M = sum(sizes)
    x = (torch.randn(M, 72, generator=g, device=gpu) * 3).to(torch.bfloat16)
    ends = workloads.ends_of(sizes)
    qt, st, pad = ops.to_mxfp8_dim1(x, torch.from_numpy(ends).to(gpu), mode | enc)
    cap = qt.shape[1]
    rq, rs, rpad = O.quant_dim1(bits(x), ends, cap, mode)
    assert np.array_equal(pad.cpu().numpy(), rpad)
    assert np.array_equal(u8(qt), rq)
    assert np.array_equal(u8(st), rs)


def test_dim1_ungrouped_and_torchao_layout(gpu):
    g = torch.Generator(device=gpu).manual_seed(16)
    x = torch.randn(96, 64, generator=g, device=gpu).to(torch.bfloat16)
    qt, st, pad = ops.to_mxfp8_dim1(x)
    assert pad is None and qt.shape == (64, 96)
    rq, rs, _ = O.quant_dim1(bits(x), None, 96, O.RCEIL)
    assert np.array_equal(u8(qt), rq) and np.array_equal(u8(st), rs)
    d, sc = mxfp8gg.triton_to_mxfp8_dim1(x, scaling_mode="rceil")
    assert d.shape == (96, 64) and d.stride() == (1, 96)   # column-major [M, K]
    assert torch.equal(d.t().view(torch.uint8), qt.view(torch.uint8))
    assert torch.equal(sc.view(torch.uint8), st)
    assert sc.is_contiguous() and sc.shape == (64, 3)     # torchao's contiguous scales
    d0, s0 = mxfp8gg.triton_to_mxfp8_dim0(x, scaling_mode="floor")
    rq0, rs0 = O.quant_dim0(bits(x), O.FLOOR)
    assert np.array_equal(u8(d0), rq0) and np.array_equal(u8(s0), rs0)
    assert s0.is_contiguous() and s0.view(-1).numel() == 96 * 2
    # the block-major view on request, same bytes
    _, s0b = mxfp8gg.triton_to_mxfp8_dim0(x, scaling_mode="floor", scale_layout="block")
    assert s0b.stride(0) == 1 and torch.equal(s0b.view(torch.uint8), s0.view(torch.uint8))


@pytest.mark.parametrize("shape", [(3, 40, 128), (77, 64)])
def test_row_major_scale_layout_option(gpu, shape):
    g = torch.Generator(device=gpu).manual_seed(17)
    x = torch.randn(*shape, generator=g, device=gpu).to(torch.bfloat16)
    q, s = ops.to_mxfp8_dim0(x)
    qr, sr = ops.to_mxfp8_dim0(x, scale_layout="row")
    assert sr.is_contiguous() and sr.shape == s.shape
    assert torch.equal(q.view(torch.uint8), qr.view(torch.uint8)) and torch.equal(s, sr)
    x2 = x.reshape(-1, shape[-1])
    ends = torch.tensor([x2.shape[0] // 3, x2.shape[0]], dtype=torch.int32, device=gpu)
    qt, st, pad = ops.to_mxfp8_dim1(x2, ends)
    qtr, str_, padr = ops.to_mxfp8_dim1(x2, ends, scale_layout="row")
    assert str_.is_contiguous() and str_.shape == st.shape
    assert torch.equal(qt.view(torch.uint8), qtr.view(torch.uint8)) and torch.equal(st, str_)
    assert torch.equal(pad, padr)
    with pytest.raises(ValueError, match="scale_layout"):
        ops.to_mxfp8_dim0(x, scale_layout="col")


def test_dim1_nan_inf_blocks(gpu):
    x = torch.randn(64, 16, device=gpu).to(torch.bfloat16)
    x[3, 2] = float("nan")
    x[40, 5] = float("inf")
    x[41, 6] = -float("inf")
    ends = np.array([20, 64], dtype=np.int32)
    for mode in (O.RCEIL, O.FLOOR):
        qt, st, _ = ops.to_mxfp8_dim1(x, torch.from_numpy(ends).to(gpu), mode)
        rq, rs, _ = O.quant_dim1(bits(x), ends, qt.shape[1], mode)
        assert np.array_equal(u8(qt), rq) and np.array_equal(u8(st), rs)


def test_dim1_c4_sampled_features(gpu):
    dy, x, sizes = workloads.c4(gpu)
    ends = workloads.ends_of(sizes)
    feats = np.array([0, 1, 777, 4095])
    qt, st, pad = ops.to_mxfp8_dim1(dy, torch.from_numpy(ends).to(gpu))
    cap = qt.shape[1]
    rq, rs, rpad = O.quant_dim1(bits(dy[:, torch.from_numpy(feats).to(gpu)]), ends, cap, O.RCEIL)
    idx = torch.from_numpy(feats).to(gpu)
    assert np.array_equal(pad.cpu().numpy(), rpad)
    assert np.array_equal(u8(qt[idx]), rq) and np.array_equal(u8(st[idx]), rs)


def test_dim1_past_the_grid_y_range_equals_transposed_dim0(gpu):
    # 2^23 tokens: 65536 blocks of 128 positions, one more than the grid's y
    # range, so the cast takes its positions-fastest grid.  One group: the
    # token-axis cast is then the row-wise cast of x transposed (independent
    # kernel, itself pinned against the oracle above).
    M, C = 1 << 23, 32
    g = torch.Generator(device=gpu).manual_seed(18)
    x = torch.randn(M, C, generator=g, device=gpu).to(torch.bfloat16)
    qt, st, pad = ops.to_mxfp8_dim1(x)
    assert pad is None and qt.shape == (C, M) and (M + 127) // 128 > 65535
    q0, s0 = ops.to_mxfp8_dim0(x.t().contiguous())
    assert torch.equal(qt.view(torch.uint8), q0.view(torch.uint8))
    assert torch.equal(st, s0)


# ---------------------------------------------------------------------------
# dual cast: both casts of one tensor from a single read
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("name,mode", MODES)
@pytest.mark.parametrize("enc", ENCODERS)
@pytest.mark.parametrize("sizes,cols", [([5, 0, 64, 33, 1, 40, 0], 96), ([128, 128], 64),
                                        ([300], 288), ([0, 0, 7], 32)])
def test_dual_matches_oracle(gpu, name, mode, enc, sizes, cols):
    g = torch.Generator(device=gpu).manual_seed(17)
    M = sum(sizes)
    x = torch.randn(M, cols, generator=g, device=gpu) * 3
    x = x * torch.exp2(torch.randint(-40, 40, (M, 1), generator=g, device=gpu).float())
    if M > 50:
        x[3, 2] = float("nan")
        x[40, 5] = float("inf")
        x[41, cols - 1] = -float("inf")
    x = x.to(torch.bfloat16)
    ends = workloads.ends_of(sizes)
    q, s, qt, st, pad = ops.to_mxfp8_dual(x, torch.from_numpy(ends).to(gpu), mode | enc)
    rq, rs = O.quant_dim0(bits(x), mode)
    assert np.array_equal(u8(q), rq) and np.array_equal(u8(s), rs)
    rqt, rst, rpad = O.quant_dim1(bits(x), ends, qt.shape[1], mode)
    assert np.array_equal(pad.cpu().numpy(), rpad)
    assert np.array_equal(u8(qt), rqt) and np.array_equal(u8(st), rst)


def test_dual_ungrouped_and_partial_groups(gpu):
    g = torch.Generator(device=gpu).manual_seed(18)
    x = torch.randn(100, 64, generator=g, device=gpu).to(torch.bfloat16)
    q, s, qt, st, pad = ops.to_mxfp8_dual(x)
    assert pad is None
    rq, rs = O.quant_dim0(bits(x), O.RCEIL)
    assert np.array_equal(u8(q), rq) and np.array_equal(u8(s), rs)
    rqt, rst, _ = O.quant_dim1(bits(x), None, qt.shape[1], O.RCEIL)
    assert np.array_equal(u8(qt), rqt) and np.array_equal(u8(st), rst)
    # groups ending before the last row: row-wise rows inside the groups only
    ends = np.array([10, 10, 70], dtype=np.int32)
    q, s, qt, st, pad = ops.to_mxfp8_dual(x, torch.from_numpy(ends).to(gpu))
    assert np.array_equal(u8(q[:70]), rq[:70]) and np.array_equal(u8(s[:70]), rs[:70])
    rqt, rst, _ = O.quant_dim1(bits(x), ends, qt.shape[1], O.RCEIL)
    assert np.array_equal(u8(qt), rqt) and np.array_equal(u8(st), rst)


@pytest.mark.parametrize("name,mode", MODES)
def test_quant_weight_dual_equals_separate_casts(gpu, name, mode):
    g = torch.Generator(device=gpu).manual_seed(19)
    w = (torch.randn(3, 64, 96, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    (wq, ws), (wt, wts) = mxfp8gg.quant_weight_dual(w, mode)
    q0, s0 = ops.to_mxfp8_dim0(w, mode)
    t0, ts0 = mxfp8gg.quant_weight_for_dgrad(w, mode)
    assert wq.shape == q0.shape and ws.shape == s0.shape
    assert wt.shape == t0.shape and wts.shape == ts0.shape
    assert np.array_equal(u8(wq), u8(q0)) and np.array_equal(u8(ws), u8(s0))
    assert np.array_equal(u8(wt), u8(t0)) and np.array_equal(u8(wts), u8(ts0))


def test_dual_c2_activation_full_size(gpu):
    # full C2 activation: byte-identical to the two single casts (each pinned
    # against the oracle above)
    x, w, sizes = workloads.c2(gpu)
    del w
    e = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    q, s, qt, st, pad = ops.to_mxfp8_dual(x, e)
    q0, s0 = ops.to_mxfp8_dim0(x)
    qt1, st1, pad1 = ops.to_mxfp8_dim1(x, e)
    assert torch.equal(q.view(torch.uint8), q0.view(torch.uint8))
    assert torch.equal(s.contiguous(), s0.contiguous())
    assert torch.equal(qt.view(torch.uint8), qt1.view(torch.uint8))
    assert torch.equal(st.contiguous(), st1.contiguous())
    assert torch.equal(pad, pad1)
