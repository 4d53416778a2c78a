"""GPU parity of the grouped GEMMs against the CPU oracle.

Tolerance (see tests/_helpers.assert_close_to_oracle): every element within
2^-7 |ref| + 2^-12 max|ref| of the float64 dequantise-then-matmul reference,
and max|err| / max|ref| <= 1e-2.  Known-answer tests are exact.
"""
import numpy as np
import pytest
import torch

import fused_fwd
import fwd_final
import mxfp8gg
import wgrad_fused
from mxfp8gg import ops, workloads
from oracle import oracle as O
from tests._helpers import assert_close_to_oracle, bits, fp8_dev, u8

pytestmark = pytest.mark.gpu


def _ones(shape, gpu):
    return torch.ones(shape, device=gpu, dtype=torch.bfloat16).to(torch.float8_e4m3fn)


# ---------------------------------------------------------------------------
# the reference's E8M0 known-answer tests (scale_correctness.py), called with
# the reference's argument forms ([E+1] offs with leading 0, tile kwargs)
# ---------------------------------------------------------------------------
def test_kat_scale_bypass(gpu):
    M, N, K, E = 64, 32, 64, 2
    a_s = torch.full((M, K // 32), 127, dtype=torch.uint8, device=gpu)
    a_s[:, 0] = 128
    w_s = torch.full((E, N, K // 32), 127, dtype=torch.uint8, device=gpu)
    offs = torch.tensor([0, M // 2, M], dtype=torch.int32, device=gpu)
    c = fused_fwd.fused_grouped_fwd(_ones((M, K), gpu), _ones((E, N, K), gpu), offs,
                                    a_scales=a_s, w_scales=w_s, BLOCK_M=64, BLOCK_N=32,
                                    BLOCK_K=64, GROUP_SIZE_M=1)
    assert c.dtype == torch.bfloat16 and torch.all(c.float() == 96.0)


def test_kat_scale_application_order(gpu):
    M, N, K = 64, 32, 64
    a_s = torch.full((M, 2), 127, dtype=torch.uint8, device=gpu)
    a_s[:, 0], a_s[:, 1] = 128, 126
    w_s = torch.full((1, N, 2), 127, dtype=torch.uint8, device=gpu)
    w_s[:, :, 0] = 129
    offs = torch.tensor([0, M], dtype=torch.int32, device=gpu)
    c = fused_fwd.fused_grouped_fwd(_ones((M, K), gpu), _ones((1, N, K), gpu), offs,
                                    a_scales=a_s, w_scales=w_s)
    assert torch.all(c.float() == 272.0)


def test_kat_scale_layout_every_row(gpu):
    M, N, K = 64, 32, 64
    a_s = torch.full((M, 2), 127, dtype=torch.uint8, device=gpu)
    a_s[:, 0] = torch.clamp(127 + torch.arange(M, device=gpu), max=254).to(torch.uint8)
    w_s = torch.full((1, N, 2), 127, dtype=torch.uint8, device=gpu)
    c = fused_fwd.fused_grouped_fwd(_ones((M, K), gpu), _ones((1, N, K), gpu),
                                    torch.tensor([0, M], dtype=torch.int32, device=gpu),
                                    a_scales=a_s, w_scales=w_s, out_dtype=torch.float32)
    expect = 32.0 * torch.exp2(torch.arange(M, dtype=torch.float64)) + 32.0
    got = c.double().cpu()
    # exact while representable in fp32 (m < 20), then within fp32 rounding
    assert torch.equal(got[:20], expect[:20, None].expand(20, N))
    assert torch.allclose(got, expect[:, None].expand(M, N), rtol=2 ** -23, atol=0)


def test_kat_per_column_and_per_block_scales(gpu):
    # W-side layout: column n gets 2^(n%8) on block b=n%4 — catches a transposed
    # or shifted B-scale lane mapping the reference's KATs leave open.
    M, N, K = 32, 64, 128
    w_s = torch.full((1, N, 4), 127, dtype=torch.uint8, device=gpu)
    n = torch.arange(N, device=gpu)
    w_s[0, n, n % 4] = (127 + n % 8).to(torch.uint8)
    a_s = torch.full((M, 4), 127, dtype=torch.uint8, device=gpu)
    c = ops.grouped_mm(_ones((M, K), gpu), _ones((1, N, K), gpu), None, a_s, w_s,
                       out_dtype=torch.float32)
    expect = 96.0 + 32.0 * torch.exp2((n % 8).double())
    assert torch.equal(c.double(), expect[None, :].expand(M, N))


def test_kat_scale_pairs_with_its_own_32_elements(gpu):
    # Row data: k-block 0 all 1.0, k-block 1 all 0; A scales 2^3 / 2^0.  Only a
    # kernel that applies each scale to exactly its own 32 contiguous elements
    # gives 32 * 8 = 256 (pairing half-blocks would give 16*8 + 16*1 = 144).
    M, N, K = 32, 32, 64
    a = torch.zeros((M, K), dtype=torch.bfloat16, device=gpu)
    a[:, :32] = 1.0
    a_s = torch.full((M, 2), 127, dtype=torch.uint8, device=gpu)
    a_s[:, 0] = 130
    w_s = torch.full((1, N, 2), 127, dtype=torch.uint8, device=gpu)
    c = ops.grouped_mm(a.to(torch.float8_e4m3fn), _ones((1, N, K), gpu), None, a_s, w_s,
                       out_dtype=torch.float32)
    assert torch.all(c == 256.0)
    # same on the W side, block 1 carrying the data
    w = torch.zeros((1, N, K), dtype=torch.bfloat16, device=gpu)
    w[:, :, 32:] = 1.0
    w_s[:, :, 1] = 125
    c = ops.grouped_mm(_ones((M, K), gpu), w.to(torch.float8_e4m3fn), None,
                       torch.full((M, 2), 127, dtype=torch.uint8, device=gpu), w_s,
                       out_dtype=torch.float32)
    assert torch.all(c == 8.0)


# ---------------------------------------------------------------------------
# random data against the oracle
# ---------------------------------------------------------------------------
def _rand_q(shape, gpu, seed, scale_lo=118, scale_hi=136):
    g = torch.Generator(device=gpu).manual_seed(seed)
    codes = torch.randint(0, 0x7E, shape, generator=g, device=gpu, dtype=torch.int32)
    sign = torch.randint(0, 2, shape, generator=g, device=gpu, dtype=torch.int32) << 7
    q = (codes | sign).to(torch.uint8)
    s_shape = shape[:-1] + (shape[-1] // 32,)
    s = torch.randint(scale_lo, scale_hi, s_shape, generator=g, device=gpu,
                      dtype=torch.int32).to(torch.uint8)
    return q, s


@pytest.mark.parametrize("sizes,N,K", [
    ([64, 128, 32, 96], 512, 256),          # C1 geometry
    ([0, 300, 1, 0, 212], 384, 320),        # empty groups, N and K tails (K % 128 = 64)
    ([513], 256, 128),                      # one group, M tail
    ([256, 256, 256], 256, 1024),           # aligned, several K stages
    ([7, 0, 0], 96, 32),                    # tiny
    ([3, 5, 9, 250], 320, 192),             # group starts not multiples of 4, odd stage count
])
@pytest.mark.parametrize("scaled", [True, False])
def test_grouped_fwd_random_codes(gpu, sizes, N, K, scaled):
    E, M = len(sizes), sum(sizes)
    a_q, a_s = _rand_q((M, K), gpu, 21)
    w_q, w_s = _rand_q((E, N, K), gpu, 22)
    ends = workloads.ends_of(sizes)
    y = ops.grouped_mm(a_q.view(torch.float8_e4m3fn), w_q.view(torch.float8_e4m3fn),
                       torch.from_numpy(ends).to(gpu), a_s if scaled else None,
                       w_s if scaled else None)
    ref = O.grouped_fwd(u8(a_q), u8(a_s) if scaled else None, u8(w_q),
                        u8(w_s) if scaled else None, ends)
    assert_close_to_oracle(y, ref)


def test_scale_layouts_give_identical_results(gpu):
    # block-major views (the cast's own output), row-major copies (re-laid by
    # the converter kernel) and per-expert block-major buffers built by hand
    x, w, sizes = workloads.c1(gpu)
    xq, xs = mxfp8gg.to_mxfp8_dim0(x)
    wq, ws = mxfp8gg.to_mxfp8_dim0(w)
    ends = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    y_view = ops.grouped_mm(xq, wq, ends, xs, ws, out_dtype=torch.float32)
    y_rm = ops.grouped_mm(xq, wq, ends, xs.contiguous(), ws.contiguous(), out_dtype=torch.float32)
    ws_sep = torch.empty((4, 8, 528), dtype=torch.uint8, device=gpu)
    ws_sep[:, :, :512] = ws.contiguous().transpose(1, 2)
    y_sep = ops.grouped_mm(xq, wq, ends, xs, ws_sep[:, :, :512].transpose(1, 2),
                           out_dtype=torch.float32)
    assert torch.equal(y_view, y_rm) and torch.equal(y_view, y_sep)


@pytest.mark.parametrize("batch,rows,nblk", [(1, 300, 7), (3, 64, 224), (2, 1, 1), (1, 4096, 2)])
def test_scales_to_block_major_kernel(gpu, batch, rows, nblk):
    from mxfp8gg import _lib

    g = torch.Generator(device=gpu).manual_seed(71)
    src = torch.randint(0, 256, (batch, rows, nblk), generator=g, device=gpu,
                        dtype=torch.int32).to(torch.uint8)
    ld = (rows + 15) // 16 * 16
    dst = torch.zeros((batch, nblk, ld), dtype=torch.uint8, device=gpu)
    lib = _lib.load()
    _lib.check(lib.mxgg_scales_to_block_major(src.data_ptr(), batch, rows, nblk, rows * nblk,
                                              nblk, dst.data_ptr(), nblk * ld, ld,
                                              torch.cuda.current_stream().cuda_stream), "t")
    assert torch.equal(dst[:, :, :rows], src.transpose(1, 2))
    assert torch.all(dst[:, :, rows:] == 0)


def test_c1_end_to_end_quant_then_gemm(gpu):
    x, w, sizes = workloads.c1(gpu)
    xq, xs = mxfp8gg.to_mxfp8_dim0(x)
    wq, ws = mxfp8gg.to_mxfp8_dim0(w)
    ends = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    y = fused_fwd.fused_grouped_fwd(xq, wq, ends, xs, ws)
    ref = O.grouped_fwd(u8(xq), u8(xs), u8(wq), u8(ws), workloads.ends_of(sizes))
    assert_close_to_oracle(y, ref)
    # and the dequant path matches the unquantised bf16 product to MXFP8 accuracy
    bf = torch.cat([x[b:e].float() @ w[g].float().T
                    for g, (b, e) in enumerate(O.group_bounds(workloads.ends_of(sizes), 320))])
    assert (y.float() - bf).abs().max() / bf.abs().max() < 0.1


def test_rows_outside_groups_untouched_and_each_row_written(gpu):
    sizes = [100, 0, 37]
    M, N, K = 200, 256, 128
    a_q, a_s = _rand_q((M, K), gpu, 31)
    w_q, w_s = _rand_q((3, N, K), gpu, 32)
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
    ops.grouped_mm(a_q.view(torch.float8_e4m3fn), w_q.view(torch.float8_e4m3fn),
                   torch.tensor(np.cumsum(sizes), dtype=torch.int32, device=gpu), a_s, w_s,
                   out=out)
    assert not torch.isnan(out[:137]).any()
    assert torch.isnan(out[137:]).all()


@pytest.mark.parametrize("scaled", [True, False])
def test_rows_past_the_last_group_never_reach_the_output(gpu, scaled):
    # A's rows past the last group end hold NaN codes (0x7F) and NaN scales
    # (0xFF); the last group's partial m-tile spans them.  Every row inside a
    # group matches the oracle on the clean rows, and the rows past the end
    # keep the sentinel.
    sizes = [100, 37]
    M, N, K = 300, 256, 256
    a_q, a_s = _rand_q((M, K), gpu, 33)
    w_q, w_s = _rand_q((2, N, K), gpu, 34)
    a_q[137:] = 0x7F
    a_s[137:] = 0xFF
    ends = workloads.ends_of(sizes)
    out = torch.full((M, N), 7.0, dtype=torch.bfloat16, device=gpu)
    ops.grouped_mm(a_q.view(torch.float8_e4m3fn), w_q.view(torch.float8_e4m3fn),
                   torch.from_numpy(ends).to(gpu), a_s if scaled else None,
                   w_s if scaled else None, out=out)
    ref = O.grouped_fwd(u8(a_q[:137]), u8(a_s[:137]) if scaled else None, u8(w_q),
                        u8(w_s) if scaled else None, ends)
    assert_close_to_oracle(out[:137], ref)
    assert torch.all(out[137:] == 7.0)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("col0,pad", [(0, 8), (0, 4), (4, 4)])
def test_output_inside_a_wider_buffer(gpu, out_dtype, col0, pad):
    """out as a column slice of a wider buffer.  Waves whose rows and columns
    lie inside the output store through one buffer range at the output's row
    stride when rows start 16-byte aligned; bf16 rows off that alignment (pad 4
    makes the stride 8 mod 16 bytes, col0 4 moves the base) and the waves at
    ragged group ends or the last column tile (N = 576) take the guarded
    stores.  Every layout gives the contiguous result bit for bit and leaves
    the columns outside [col0, col0 + N) untouched."""
    sizes = [300, 0, 700, 25]
    M, N, K = sum(sizes), 576, 256
    a_q, a_s = _rand_q((M, K), gpu, 41)
    w_q, w_s = _rand_q((len(sizes), N, K), gpu, 42)
    ends = torch.tensor(np.cumsum(sizes), dtype=torch.int32, device=gpu)
    args = (a_q.view(torch.float8_e4m3fn), w_q.view(torch.float8_e4m3fn), ends, a_s, w_s)
    ref = ops.grouped_mm(*args, out_dtype=out_dtype)
    big = torch.full((M, col0 + N + pad), float("nan"), dtype=out_dtype, device=gpu)
    got = ops.grouped_mm(*args, out_dtype=out_dtype, out=big[:, col0:col0 + N])
    assert torch.equal(got.contiguous().view(torch.uint8), ref.view(torch.uint8))
    assert torch.isnan(big[:, :col0]).all() and torch.isnan(big[:, col0 + N:]).all()


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("N", [4, 20, 100, 276])
def test_forward_column_count_off_the_8_grid(gpu, N, out_dtype, split):
    """N = 4 mod 8 (one or two column tiles): bf16 output rows start off
    16-byte alignment and the last column tile ends inside a 16-byte chunk,
    so those columns leave through the per-element stores, from the GEMM's
    epilogue or from the split-K reduce."""
    sizes = [40, 0, 300, 13]
    M, K = sum(sizes), 512                  # 4 stages: the split entry cuts them
    a_q, a_s = _rand_q((M, K), gpu, 61)
    w_q, w_s = _rand_q((len(sizes), N, K), gpu, 62)
    ends = workloads.ends_of(sizes)
    y = ops.grouped_mm(a_q.view(torch.float8_e4m3fn), w_q.view(torch.float8_e4m3fn),
                       torch.from_numpy(ends).to(gpu), a_s, w_s, out_dtype=out_dtype,
                       split_tail=split)
    ref = O.grouped_fwd(u8(a_q), u8(a_s), u8(w_q), u8(w_s), ends)
    assert_close_to_oracle(y, ref)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("N", [1, 6, 17, 259])
def test_forward_any_column_count(gpu, N, out_dtype, split):
    """Column counts off the 4-element grid (the reference masks any N,
    fused_fwd.py:163-164): the output runs at a padded row stride and comes
    back contiguous, equal to the oracle, through grouped_mm and the drop-in
    fused_grouped_fwd."""
    sizes = [40, 0, 300, 13]
    M, K = sum(sizes), 256
    a_q, a_s = _rand_q((M, K), gpu, 63)
    w_q, w_s = _rand_q((len(sizes), N, K), gpu, 64)
    ends = workloads.ends_of(sizes)
    args = (a_q.view(torch.float8_e4m3fn), w_q.view(torch.float8_e4m3fn),
            torch.from_numpy(ends).to(gpu), a_s, w_s)
    y = ops.grouped_mm(*args, out_dtype=out_dtype, split_tail=split)
    assert y.shape == (M, N) and y.is_contiguous()
    ref = O.grouped_fwd(u8(a_q), u8(a_s), u8(w_q), u8(w_s), ends)
    assert_close_to_oracle(y, ref)
    if out_dtype == torch.bfloat16 and not split:
        y2 = fused_fwd.fused_grouped_fwd(*args)
        assert y2.shape == (M, N) and y2.is_contiguous()
        assert_close_to_oracle(y2, ref)


def test_scale_bump_doubles_output_exactly(gpu):
    x, w, sizes = workloads.c1(gpu)
    xq, xs = mxfp8gg.to_mxfp8_dim0(x)
    wq, ws = mxfp8gg.to_mxfp8_dim0(w)
    ends = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    y = ops.grouped_mm(xq, wq, ends, xs, ws, out_dtype=torch.float32)
    y2 = ops.grouped_mm(xq, wq, ends, xs + 1, ws, out_dtype=torch.float32)
    assert torch.equal(y2, 2 * y)


def test_fwd_ge_dense(gpu):
    g = torch.Generator(device=gpu).manual_seed(41)
    M, K, N = 300, 256, 320
    x = torch.randn(M, K, generator=g, device=gpu).to(torch.float8_e4m3fn)
    w_nk = torch.randn(N, K, generator=g, device=gpu).to(torch.float8_e4m3fn)
    ref = O.grouped_fwd(u8(x), None, u8(w_nk)[None], None, None)
    y1 = fwd_final.fwd_ge(x, w_nk.t().contiguous())     # [K, N] row-major
    y2 = fwd_final.fwd_ge(x, w_nk.t())                   # transposed view, no copy
    assert_close_to_oracle(y1, ref)
    assert torch.equal(y1, y2)


def test_torchao_named_forward(gpu):
    x, w, sizes = workloads.c1(gpu)
    xq, xs = mxfp8gg.triton_to_mxfp8_dim0(x, scaling_mode="rceil")
    wq, ws = mxfp8gg.triton_to_mxfp8_dim0(w, scaling_mode="rceil")
    ends = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    y1 = mxfp8gg.triton_mxfp8_grouped_mm(xq, wq, xs, ws, ends)
    y2 = mxfp8gg.triton_mxfp8_grouped_mm(xq, wq.transpose(-2, -1), xs, ws, ends)
    y3 = fused_fwd.fused_grouped_fwd(xq, wq, ends, xs, ws)
    assert torch.equal(y1, y2) and torch.equal(y1, y3)


def test_forward_above_2gib_runs_in_row_chunks(gpu):
    # A is 360000 x 7168 e4m3 = 2.58 GB, past the 32-bit buffer range of one
    # launch: grouped_mm runs it as row chunks of 299520 rows with shifted
    # group ends.  The C ABI refuses the whole matrix in one launch; rows at
    # the chunk boundary, at group boundaries and at both ends match the
    # oracle, and one group straddles the chunk boundary.
    M, N, K = 360000, 256, 7168
    sizes = [100000, 250000, 10000]
    g = torch.Generator(device=gpu).manual_seed(51)
    a = torch.randint(0, 0x7E, (M, K), generator=g, device=gpu, dtype=torch.uint8)
    a |= torch.randint(0, 2, (M, K), generator=g, device=gpu, dtype=torch.uint8) << 7
    a_s = torch.randint(120, 134, (M, K // 32), generator=g, device=gpu, dtype=torch.uint8)
    w = torch.randint(0, 0x7E, (3, N, K), generator=g, device=gpu, dtype=torch.uint8)
    w_s = torch.randint(120, 134, (3, N, K // 32), generator=g, device=gpu, dtype=torch.uint8)
    assert ops._rows_per_launch(K, K, M) == 299520
    ends = torch.tensor(np.cumsum(sizes), dtype=torch.int32, device=gpu)
    f8 = torch.float8_e4m3fn
    y = ops.grouped_mm(a.view(f8), w.view(f8), ends, a_s, w_s)
    lib = mxfp8gg.load_library()
    assert lib.mxgg_grouped_fwd(a.data_ptr(), K, None, 0, w.data_ptr(), N * K, K, None, 0, 0,
                                ends.data_ptr(), 3, M, N, K, y.data_ptr(), N, 0,
                                None) == mxfp8gg._lib.ERR_UNSUPPORTED
    rows = np.r_[0:8, 99990:100010, 299500:299540, 349990:350010, M - 8:M]
    ri = torch.from_numpy(rows).to(gpu)
    grp = np.searchsorted(np.cumsum(sizes), rows, side="right")
    for e in range(3):
        sel = rows[grp == e]
        if sel.size == 0:
            continue
        si = torch.from_numpy(sel).to(gpu)
        ref = O.grouped_fwd(u8(a[si]), u8(a_s[si]), u8(w[e:e + 1]), u8(w_s[e:e + 1]),
                            np.array([sel.size]))
        assert_close_to_oracle(y[si], ref)
    assert not torch.isnan(y[ri].float()).any()


def test_wgrad_above_2gib_runs_in_feature_row_chunks(gpu):
    # dY^T and X^T of 300032 padded tokens x 7168 features are 2.15 GB each,
    # past the 32-bit buffer range of one launch: grouped_wgrad runs 2 x 2
    # launches over chunks of 6912 feature rows of each operand, each writing
    # its slice of dW (mxgg_grouped_wgrad_strided).  The C ABI refuses the
    # whole operand in one launch; sampled dW entries on both sides of both
    # chunk boundaries match the oracle for every expert.
    N = K = 7168
    M = 300032
    sizes = [100032, 0, 170016, 29984]          # multiples of 32, an empty expert
    g = torch.Generator(device=gpu).manual_seed(57)

    def operand(rows):
        q = torch.randint(0, 0x7E, (rows, M), generator=g, device=gpu, dtype=torch.uint8)
        q |= torch.randint(0, 2, (rows, M), generator=g, device=gpu, dtype=torch.uint8) << 7
        s = torch.randint(120, 134, (M // 32, rows), generator=g, device=gpu, dtype=torch.uint8)
        return q, s.t()                        # scales as a block-major view [rows, M/32]

    go, gos = operand(N)
    ia, ias = operand(K)
    assert ops._feature_rows_per_launch(M, N, M) == 6912
    ends = torch.tensor(np.cumsum(sizes), dtype=torch.int32, device=gpu)
    f8 = torch.float8_e4m3fn
    lib = mxfp8gg.load_library()
    dw_one = torch.empty((4, N, K), dtype=torch.float32, device=gpu)
    assert lib.mxgg_grouped_wgrad(go.data_ptr(), M, gos.data_ptr(), N, ia.data_ptr(), M,
                                  ias.data_ptr(), K, ends.data_ptr(), 4, M, N, K,
                                  dw_one.data_ptr(), 1, 0, None) == mxfp8gg._lib.ERR_UNSUPPORTED
    del dw_one
    dw = ops.grouped_wgrad(go.view(f8), ia.view(f8), ends, gos, ias, out_dtype=torch.float32)
    pick = np.array([0, 255, 6911, 6912, 7000, 7167])
    pi = torch.from_numpy(pick).to(gpu)
    ref = O.grouped_wgrad(u8(go[pi]), u8(gos[pi]), u8(ia[pi]), u8(ias[pi]), np.cumsum(sizes))
    got = dw[:, pi][:, :, pi]
    for e, sz in enumerate(sizes):
        if sz:
            assert_close_to_oracle(got[e], ref[e])
        else:
            assert torch.all(dw[e] == 0)


@pytest.mark.parametrize("cfg", ["c2", "c3"])
def test_full_size_forward_sampled_rows(gpu, cfg):
    x, w, sizes = getattr(workloads, cfg)(gpu)
    xq, xs = mxfp8gg.to_mxfp8_dim0(x)
    wq, ws = mxfp8gg.to_mxfp8_dim0(w)
    del x, w
    ends_np = workloads.ends_of(sizes)
    ends = torch.from_numpy(ends_np).to(gpu)
    y = ops.grouped_mm(xq, wq, ends, xs, ws)
    y_again = ops.grouped_mm(xq, wq, ends, xs, ws)
    assert torch.equal(y, y_again)  # deterministic
    # every non-empty expert: its first and last row and two random rows
    rng = np.random.default_rng(61)
    checked = 0
    for g, (b, e) in enumerate(O.group_bounds(ends_np, xq.shape[0])):
        if e <= b:
            continue
        rows = np.unique(np.r_[b, e - 1, rng.integers(b, e, 2)])
        idx = torch.from_numpy(rows).to(gpu)
        ref = O.dequant(u8(xq[idx]), u8(xs[idx])) @ O.dequant(u8(wq[g]), u8(ws[g])).T
        assert_close_to_oracle(y[idx], ref)
        checked += 1
    assert checked == int(np.count_nonzero(sizes))


@pytest.mark.parametrize("scaled", [True, False])
def test_nan_row_inside_a_group_is_compared(gpu, scaled):
    # A NaN payload code inside a group makes that output row NaN in the
    # oracle; the comparison covers it (only the rows outside every group are
    # masked out, by oracle.rows_in_groups) and the kernel gives NaN there too.
    sizes = [100, 0, 37]
    M, N, K = 200, 256, 128
    a_q, a_s = _rand_q((M, K), gpu, 35)
    w_q, w_s = _rand_q((3, N, K), gpu, 36)
    a_q[42, 5] = 0x7F
    ends = workloads.ends_of(sizes)
    out = torch.full((M, N), 7.0, dtype=torch.float32, device=gpu)
    ops.grouped_mm(a_q.view(torch.float8_e4m3fn), w_q.view(torch.float8_e4m3fn),
                   torch.from_numpy(ends).to(gpu), a_s if scaled else None,
                   w_s if scaled else None, out_dtype=torch.float32, out=out)
    ref = O.grouped_fwd(u8(a_q), u8(a_s) if scaled else None, u8(w_q),
                        u8(w_s) if scaled else None, ends)
    mask = O.rows_in_groups(ends, M)
    assert np.isnan(ref[42]).all() and mask.sum() == 137
    assert_close_to_oracle(out, ref, rows=mask)
    assert torch.all(out[torch.from_numpy(~mask).to(gpu)] == 7.0)


# ---------------------------------------------------------------------------
# wgrad
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("sizes,N,K", [
    ([64, 0, 96, 32], 256, 256),            # empty expert, aligned
    ([32, 160, 0, 0, 416], 320, 288),       # group starts not 128-aligned, N/K tails
    ([1024], 128, 512),                     # one long group, several stages
])
@pytest.mark.parametrize("scaled", [True, False])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_wgrad_random_codes(gpu, sizes, N, K, scaled, out_dtype):
    M = sum(sizes)
    go_q, go_s = _rand_q((N, M), gpu, 51)
    ia_q, ia_s = _rand_q((K, M), gpu, 52)
    ends = workloads.ends_of(sizes)
    dw = ops.grouped_wgrad(go_q.view(torch.float8_e4m3fn), ia_q.view(torch.float8_e4m3fn),
                           torch.from_numpy(ends).to(gpu), go_s if scaled else None,
                           ia_s if scaled else None, out_dtype=out_dtype)
    ref = O.grouped_wgrad(u8(go_q), u8(go_s) if scaled else None, u8(ia_q),
                          u8(ia_s) if scaled else None, ends)
    for g in range(len(sizes)):
        if sizes[g] == 0:
            assert torch.all(dw[g] == 0)
        else:
            assert_close_to_oracle(dw[g], ref[g])


def test_wgrad_reference_api_from_bf16(gpu):
    g = torch.Generator(device=gpu).manual_seed(61)
    sizes = [40, 0, 100, 7]
    M = sum(sizes)
    dy = (torch.randn(M, 192, generator=g, device=gpu) * 1e-3).to(torch.bfloat16)
    x = torch.randn(M, 160, generator=g, device=gpu).to(torch.bfloat16)
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    go, gos, pad = mxfp8gg.to_mxfp8_dim1(dy, offs)
    ia, ias, pad2 = mxfp8gg.to_mxfp8_dim1(x, offs)
    assert torch.equal(pad, pad2)
    dw = wgrad_fused.wgrad_fused(go, ia, pad, gos, ias, out_dtype=torch.float32)
    data = wgrad_fused.wgrad_prepare(go, ia, pad, gos, ias)
    assert data["E"] == 4 and data["N"] == 192 and data["K"] == 160
    dw2 = wgrad_fused.wgrad_kernel(data, out_dtype=torch.float32, BLOCK_M=128)
    assert torch.equal(dw, dw2)
    ref = O.grouped_wgrad(u8(go), u8(gos), u8(ia), u8(ias), pad.cpu().numpy())
    for e in range(4):
        if sizes[e]:
            assert_close_to_oracle(dw[e], ref[e])
        else:
            assert torch.all(dw[e] == 0)
    # bf16 default output, as in the reference
    assert wgrad_fused.wgrad_fused(go, ia, pad, gos, ias).dtype == torch.bfloat16


def test_wgrad_c4_sampled(gpu):
    dy, x, sizes = workloads.c4(gpu)
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    go, gos, pad = mxfp8gg.to_mxfp8_dim1(dy, offs)
    ia, ias, _ = mxfp8gg.to_mxfp8_dim1(x, offs)
    del dy, x
    dw = ops.grouped_wgrad(go, ia, pad, gos, ias, out_dtype=torch.float32)
    assert dw.shape == (32, 4096, 7168)
    empty = np.nonzero(sizes == 0)[0]
    assert len(empty) >= 2
    for e in empty:
        assert torch.all(dw[int(e)] == 0)
    n_rows = np.array([0, 1, 2047, 4095])
    k_rows = np.array([0, 5, 4000, 7167])
    ni, ki = torch.from_numpy(n_rows).to(gpu), torch.from_numpy(k_rows).to(gpu)
    ref = O.grouped_wgrad(u8(go[ni]), u8(gos[ni]), u8(ia[ki]), u8(ias[ki]), pad.cpu().numpy())
    got = dw[:, ni][:, :, ki]
    for e in range(32):
        if sizes[e]:
            assert_close_to_oracle(got[e], ref[e])
    # linearity in the scales: one more on every dY scale doubles dW exactly
    dw2 = ops.grouped_wgrad(go, ia, pad, gos + 1, ias, out_dtype=torch.float32)
    assert torch.equal(dw2, 2 * dw)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("split", [0, 128])
@pytest.mark.parametrize("N,K", [(36, 20), (260, 276)])
def test_wgrad_feature_counts_off_the_8_grid(gpu, N, K, out_dtype, split):
    """dW rows of K = 4 mod 8 elements (bf16 rows off 16-byte alignment, a
    last column tile ending inside a 16-byte chunk) and N = 4 mod 8 rows,
    unsplit and split along tokens (the staged partials' reduce writes them)."""
    sizes = [64, 0, 160, 32]
    M = sum(sizes)
    go_q, go_s = _rand_q((N, M), gpu, 71)
    ia_q, ia_s = _rand_q((K, M), gpu, 72)
    ends = workloads.ends_of(sizes)
    dw = ops.grouped_wgrad(go_q.view(torch.float8_e4m3fn), ia_q.view(torch.float8_e4m3fn),
                           torch.from_numpy(ends).to(gpu), go_s, ia_s, out_dtype=out_dtype,
                           split_tokens=split)
    ref = O.grouped_wgrad(u8(go_q), u8(go_s), u8(ia_q), u8(ia_s), ends)
    for g, s in enumerate(sizes):
        if s == 0:
            assert torch.all(dw[g] == 0)
        else:
            assert_close_to_oracle(dw[g], ref[g])


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("split", [0, 128])
@pytest.mark.parametrize("N,K", [(3, 1), (17, 18), (261, 259)])
def test_wgrad_any_feature_count(gpu, N, K, out_dtype, split):
    """dW rows of a K off the 4-element grid run at a padded row stride (the
    strided entry) and come back contiguous, equal to the oracle; wgrad_fused
    takes the same path."""
    sizes = [64, 0, 160, 32]
    M = sum(sizes)
    go_q, go_s = _rand_q((N, M), gpu, 73)
    ia_q, ia_s = _rand_q((K, M), gpu, 74)
    ends = workloads.ends_of(sizes)
    args = (go_q.view(torch.float8_e4m3fn), ia_q.view(torch.float8_e4m3fn),
            torch.from_numpy(ends).to(gpu), go_s, ia_s)
    dw = ops.grouped_wgrad(*args, out_dtype=out_dtype, split_tokens=split)
    assert dw.shape == (len(sizes), N, K) and dw.is_contiguous()
    ref = O.grouped_wgrad(u8(go_q), u8(go_s), u8(ia_q), u8(ia_s), ends)
    for g, s in enumerate(sizes):
        if s == 0:
            assert torch.all(dw[g] == 0)
        else:
            assert_close_to_oracle(dw[g], ref[g])
    if split == 0:
        dw2 = wgrad_fused.wgrad_fused(*args, out_dtype=out_dtype, offs_kind="ends")
        assert dw2.shape == dw.shape and dw2.is_contiguous()
        for g, s in enumerate(sizes):
            if s:
                assert_close_to_oracle(dw2[g], ref[g])


@pytest.mark.parametrize("sizes,split", [([1024, 0, 2976, 96], 256), ([4096, 4096], 1024),
                                         ([640, 32], 128)])
def test_wgrad_split_k_matches_oracle(gpu, sizes, split):
    M = sum(sizes)
    N, K = 256, 320
    go_q, go_s = _rand_q((N, M), gpu, 53)
    ia_q, ia_s = _rand_q((K, M), gpu, 54)
    ends = workloads.ends_of(sizes)
    offs = torch.from_numpy(ends).to(gpu)
    go8, ia8 = go_q.view(torch.float8_e4m3fn), ia_q.view(torch.float8_e4m3fn)
    dw = ops.grouped_wgrad(go8, ia8, offs, go_s, ia_s, out_dtype=torch.float32, split_tokens=split)
    ref = O.grouped_wgrad(u8(go_q), u8(go_s), u8(ia_q), u8(ia_s), ends)
    whole = ops.grouped_wgrad(go8, ia8, offs, go_s, ia_s, out_dtype=torch.float32, split_tokens=0)
    for g in range(len(sizes)):
        if sizes[g] == 0:
            assert torch.all(dw[g] == 0)
        else:
            assert_close_to_oracle(dw[g], ref[g])
            # same sum in another order: fp32 rounding differences only
            assert (dw[g] - whole[g]).abs().max() <= 2.0 ** -12 * whole[g].abs().max()


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_wgrad_staged_split_deterministic_any_dtype(gpu, out_dtype):
    # the workspace split (mxgg_grouped_wgrad_split): bf16 output too, no
    # zeroing of dW (a NaN-filled output comes back with zeros for the empty
    # expert), bit-equal repeat calls, the unsplit result up to fp32 summation
    # order, and the fp32-atomics split of mxgg_grouped_wgrad within the same
    # bound
    sizes = [1024, 0, 2976, 96, 352]
    M, N, K = sum(sizes), 288, 320
    go_q, go_s = _rand_q((N, M), gpu, 61)
    ia_q, ia_s = _rand_q((K, M), gpu, 62)
    ends = workloads.ends_of(sizes)
    offs = torch.from_numpy(ends).to(gpu)
    go8, ia8 = go_q.view(torch.float8_e4m3fn), ia_q.view(torch.float8_e4m3fn)
    E = len(sizes)
    out = torch.full((E, N, K), float("nan"), dtype=out_dtype, device=gpu)
    dw = ops.grouped_wgrad(go8, ia8, offs, go_s, ia_s, out_dtype=out_dtype, out=out,
                           split_tokens=256)
    dw2 = ops.grouped_wgrad(go8, ia8, offs, go_s, ia_s, out_dtype=out_dtype, split_tokens=256)
    assert torch.equal(dw.view(torch.uint8), dw2.view(torch.uint8))
    assert torch.all(dw[1] == 0)
    whole = ops.grouped_wgrad(go8, ia8, offs, go_s, ia_s, out_dtype=out_dtype, split_tokens=0)
    ref = O.grouped_wgrad(u8(go_q), u8(go_s), u8(ia_q), u8(ia_s), ends)
    tol = 2.0 ** -12 if out_dtype == torch.float32 else 2.0 ** -7
    for g in (0, 2, 3, 4):
        assert_close_to_oracle(dw[g], ref[g])
        assert (dw[g].float() - whole[g].float()).abs().max() <= tol * whole[g].float().abs().max()
    if out_dtype == torch.float32:
        sg, ldg = ops._scales_2d(go_s, N, M // 32, "go_s")
        si, ldi = ops._scales_2d(ia_s, K, M // 32, "ia_s")
        at = torch.zeros((E, N, K), dtype=torch.float32, device=gpu)
        lib = mxfp8gg.load_library()
        assert lib.mxgg_grouped_wgrad(
            go_q.data_ptr(), M, sg.data_ptr(), ldg, ia_q.data_ptr(), M, si.data_ptr(), ldi,
            offs.data_ptr(), E, M, N, K, at.data_ptr(), mxfp8gg._lib.OUT_F32, 256,
            torch.cuda.current_stream(gpu).cuda_stream) == 0
        assert (at - dw).abs().max() <= 2.0 ** -12 * dw.abs().max()


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("split", [0, 128])
def test_wgrad_without_tokens_is_zero(gpu, out_dtype, split):
    # every expert empty (no tokens routed here): dW is zeros, whatever the
    # layout of the empty operands (an empty [N, 0] tensor has row stride 1)
    N, K, E = 160, 224, 3
    go = torch.empty((N, 0), dtype=torch.uint8, device=gpu).view(torch.float8_e4m3fn)
    ia = torch.empty((K, 0), dtype=torch.uint8, device=gpu).view(torch.float8_e4m3fn)
    gs = torch.empty((N, 0), dtype=torch.uint8, device=gpu)
    is_ = torch.empty((K, 0), dtype=torch.uint8, device=gpu)
    ends = torch.zeros(E, dtype=torch.int32, device=gpu)
    out = torch.full((E, N, K), float("nan"), dtype=out_dtype, device=gpu)
    dw = ops.grouped_wgrad(go, ia, ends, gs, is_, out_dtype=out_dtype, out=out,
                           split_tokens=split)
    assert torch.all(dw == 0)


def test_wgrad_split_k_chosen_for_few_tiles(gpu):
    # 2 experts x 2 x 2 output tiles: far fewer than compute units, so the
    # call splits the 16384 tokens of each expert on its own
    sizes = [16384, 16384]
    M, N, K = sum(sizes), 512, 512
    assert ops.wgrad_split_tokens(M, N, K, 2, ops._cu_count(gpu)) > 0
    go_q, go_s = _rand_q((N, M), gpu, 55)
    ia_q, ia_s = _rand_q((K, M), gpu, 56)
    ends = workloads.ends_of(sizes)
    dw = ops.grouped_wgrad(go_q.view(torch.float8_e4m3fn), ia_q.view(torch.float8_e4m3fn),
                           torch.from_numpy(ends).to(gpu), go_s, ia_s, out_dtype=torch.float32)
    ref = O.grouped_wgrad(u8(go_q), u8(go_s), u8(ia_q), u8(ia_s), ends, n_rows=np.arange(0, N, 7),
                          k_rows=np.arange(0, K, 5))
    for g in range(2):
        assert_close_to_oracle(dw[g][::7, ::5], ref[g])


def test_wgrad_split_k_misaligned_group_is_nan(gpu):
    sizes = [1000, 1048]  # first end not a multiple of 32: both experts are NaN
    M = sum(sizes)
    go_q, go_s = _rand_q((256, M), gpu, 57)
    ia_q, ia_s = _rand_q((256, M), gpu, 58)
    dw = ops.grouped_wgrad(go_q.view(torch.float8_e4m3fn), ia_q.view(torch.float8_e4m3fn),
                           torch.from_numpy(workloads.ends_of(sizes)).to(gpu), go_s, ia_s,
                           out_dtype=torch.float32, split_tokens=256)
    assert torch.isnan(dw).all()
