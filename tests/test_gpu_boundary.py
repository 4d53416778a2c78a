"""GPU tests of the boundary rules around the grouped GEMMs, through the C ABI:

* `offs` forms of the reference-named wgrad entry points: group sizes (the
  reference's documentation, wgrad_fused.py:37, and its wgrad benchmark,
  bench_wgrad_dsv3.py:52) and cumulative ends (its layer step,
  e2e_bench.py:42,117) both give the oracle's dW for every expert;
* group ends that are not multiples of 32 in an unscaled weight gradient
  (computed exactly, token by token) and in a scaled one (NaN: a scale block
  would span two experts);
* decreasing group ends: every kernel reads them as their running maximum
  clamped to the rows, so no row belongs to two groups (oracle.group_bounds
  states the same rule; the CPU tests pin it against numpy);
* zeroing of rows past the last group end.
"""
import numpy as np
import pytest
import torch

import mxfp8gg
from mxfp8gg import ops, workloads
from oracle import oracle as O
from tests._helpers import assert_close_to_oracle, bits, u8

pytestmark = pytest.mark.gpu

F8 = torch.float8_e4m3fn


def _rand_q(shape, gpu, seed, lo=118, hi=136):
    g = torch.Generator(device=gpu).manual_seed(seed)
    codes = torch.randint(0, 0x7E, shape, generator=g, device=gpu, dtype=torch.int32)
    sign = torch.randint(0, 2, shape, generator=g, device=gpu, dtype=torch.int32) << 7
    s = torch.randint(lo, hi, shape[:-1] + (shape[-1] // 32,), generator=g, device=gpu,
                      dtype=torch.int32).to(torch.uint8)
    return (codes | sign).to(torch.uint8), s


@pytest.mark.parametrize("offs,tokens,kind,want", [
    ([96, 96, 96], 288, "auto", [96, 192, 288]),        # sizes (bench_wgrad_dsv3.py:52)
    ([96, 192, 288], 288, "auto", [96, 192, 288]),      # ends (e2e_bench.py:117)
    ([288], 288, "auto", [288]),                        # one group: both readings agree
    ([0, 200, 0, 88], 288, "auto", [0, 200, 200, 288]),  # sizes with empty experts
    ([10, 20, 30], 64, "auto", [10, 20, 30]),           # ends that leave tokens over
    ([10, 20, 30], 60, "ends", [10, 20, 30]),           # forced readings
    ([10, 20, 30], 64, "sizes", [10, 30, 60]),
])
def test_offs_to_group_ends(gpu, offs, tokens, kind, want):
    t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    got = mxfp8gg.offs_to_group_ends(t, tokens, kind)
    assert got.tolist() == want
    assert t.tolist() == offs                            # input untouched


def test_library_group_ends_are_never_read_as_sizes(gpu):
    # one expert holding every token: the padded ends [64, 64, 64, 64] add up to
    # the padded capacity (256) exactly, which the auto rule alone would read
    # as sizes
    dy = torch.randn(64, 96, device=gpu).to(torch.bfloat16)
    offs = torch.tensor([64, 64, 64, 64], dtype=torch.int32, device=gpu)
    _, _, pad = mxfp8gg.to_mxfp8_dim1(dy, offs)
    assert pad.tolist() == [64, 64, 64, 64] and mxfp8gg.padded_token_capacity(64, 4) == 256
    assert isinstance(pad, mxfp8gg.GroupEnds)
    assert mxfp8gg.offs_to_group_ends(pad, 256).tolist() == [64, 64, 64, 64]
    # copies keep the meaning: clone, a host round trip, a concatenation
    for copy in (pad.clone(), pad.cpu().to(gpu), pad.detach().contiguous(),
                 torch.cat([pad.clone()])):
        assert mxfp8gg.offs_to_group_ends(copy, 256).tolist() == [64, 64, 64, 64]
    # a plain tensor with the same values fits both readings: auto takes sizes
    plain = torch.tensor(pad.tolist(), dtype=torch.int32, device=gpu)
    assert mxfp8gg.offs_to_group_ends(plain, 256).tolist() == [64, 128, 192, 256]
    assert mxfp8gg.offs_to_group_ends(plain, 256, "ends").tolist() == [64, 64, 64, 64]


@pytest.mark.parametrize("E,mg", [(4, 512), (8, 384)])
@pytest.mark.parametrize("scaled", [False, True])
def test_reference_wgrad_call_forms(gpu, E, mg, scaled):
    # bench_wgrad_dsv3.py:41-52: go = (N, M), ia = (K, M) cast with .to(fp8),
    # offs = [mg] * E (sizes); e2e_bench.py:114-117: cumulative ends.  Both
    # must give every expert its own dW.
    from wgrad_fused import wgrad_fused, wgrad_kernel, wgrad_prepare

    N, K = 256, 320
    M = E * mg
    go, gos = _rand_q((N, M), gpu, 91)
    ia, ias = _rand_q((K, M), gpu, 92)
    go8, ia8 = go.view(F8), ia.view(F8)
    s_go, s_ia = (gos, ias) if scaled else (None, None)
    ends = (np.arange(1, E + 1) * mg).astype(np.int32)
    ref = O.grouped_wgrad(u8(go), u8(gos) if scaled else None, u8(ia),
                          u8(ias) if scaled else None, ends)
    sizes_t = torch.tensor([mg] * E, dtype=torch.int32, device=gpu)
    ends_t = torch.from_numpy(ends).to(gpu)
    outs = [wgrad_fused(go8, ia8, sizes_t, s_go, s_ia, out_dtype=torch.float32),
            wgrad_fused(go8, ia8, ends_t, s_go, s_ia, out_dtype=torch.float32),
            wgrad_kernel(wgrad_prepare(go8, ia8, sizes_t, s_go, s_ia), out_dtype=torch.float32),
            wgrad_kernel(wgrad_prepare(go8, ia8, ends_t, s_go, s_ia), out_dtype=torch.float32)]
    for dw in outs:
        assert dw.shape == (E, N, K)
        for e in range(E):
            assert_close_to_oracle(dw[e], ref[e])
        assert torch.equal(dw, outs[0])
    # the reference's default output dtype
    assert wgrad_kernel(wgrad_prepare(go8, ia8, sizes_t, s_go, s_ia)).dtype == torch.bfloat16


@pytest.mark.parametrize("sizes", [[37, 0, 150, 5, 200], [1, 1, 1, 500], [17, 15, 32, 96, 3]])
@pytest.mark.parametrize("split", [0, 128])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_unscaled_wgrad_with_any_group_ends(gpu, sizes, split, out_dtype):
    # ends off multiples of 16 and 32 (and split-K chunks starting there): exact
    M0 = sum(sizes)
    M = (M0 + 31) // 32 * 32 + 32              # trailing tokens outside every group
    N, K = 192, 288
    go, _ = _rand_q((N, M), gpu, 93)
    ia, _ = _rand_q((K, M), gpu, 94)
    ends = workloads.ends_of(sizes)
    dw = ops.grouped_wgrad(go.view(F8), ia.view(F8), torch.from_numpy(ends).to(gpu),
                           out_dtype=out_dtype, split_tokens=split)
    ref = O.grouped_wgrad(u8(go), None, u8(ia), None, ends)
    for e, s in enumerate(sizes):
        if s:
            assert_close_to_oracle(dw[e], ref[e])
        else:
            assert torch.all(dw[e] == 0)


def test_scaled_wgrad_with_misaligned_ends_is_nan(gpu):
    sizes = [40, 88, 128]                      # ends 40 and 128: expert 0 and 1 straddle blocks
    M = sum(sizes)
    go, gos = _rand_q((128, M), gpu, 95)
    ia, ias = _rand_q((160, M), gpu, 96)
    ends = workloads.ends_of(sizes)
    dw = ops.grouped_wgrad(go.view(F8), ia.view(F8), torch.from_numpy(ends).to(gpu), gos, ias,
                           out_dtype=torch.float32)
    assert torch.isnan(dw[0]).all() and torch.isnan(dw[1]).all()
    ref = O.grouped_wgrad(u8(go), u8(gos), u8(ia), u8(ias), ends)
    assert_close_to_oracle(dw[2], ref[2])


NON_MONOTONE = [[300, 100, 500, 0, 700], [700, 0, 700, 0, 700], [-5, 64, 40, 2000]]


@pytest.mark.parametrize("ends", NON_MONOTONE)
def test_forward_reads_decreasing_ends_as_running_max(gpu, ends):
    M, N, K = 700, 256, 192
    E = len(ends)
    a, a_s = _rand_q((M, K), gpu, 97)
    w, w_s = _rand_q((E, N, K), gpu, 98)
    e_np = np.array(ends, dtype=np.int32)
    out = torch.full((M, N), float("nan"), dtype=torch.float32, device=gpu)
    ops.grouped_mm(a.view(F8), w.view(F8), torch.from_numpy(e_np).to(gpu), a_s, w_s,
                   out_dtype=torch.float32, out=out)
    ref = O.grouped_fwd(u8(a), u8(a_s), u8(w), u8(w_s), e_np)
    assert_close_to_oracle(out, ref)
    covered = np.zeros(M, bool)
    for b, t in O.group_bounds(e_np, M):
        covered[b:t] = True
    assert torch.isnan(out[torch.from_numpy(~covered).to(gpu)]).all()


@pytest.mark.parametrize("ends", NON_MONOTONE)
def test_token_casts_read_decreasing_ends_as_running_max(gpu, ends):
    M, C = 700, 96
    g = torch.Generator(device=gpu).manual_seed(99)
    x = torch.randn(M, C, generator=g, device=gpu).to(torch.bfloat16)
    e_np = np.array(ends, dtype=np.int32)
    offs = torch.from_numpy(e_np).to(gpu)
    q, s, qt, st, pad = mxfp8gg.to_mxfp8_dual(x, offs)
    cap = mxfp8gg.padded_token_capacity(M, len(ends))
    rq, rs, rpad = O.quant_dim1(bits(x), e_np, cap)
    assert np.array_equal(pad.cpu().numpy(), rpad)
    assert np.array_equal(u8(qt), rq) and np.array_equal(u8(st), rs)
    assert rpad[-1] <= (M + 31 * len(ends)) // 32 * 32


@pytest.mark.parametrize("split", [0, 128])
def test_wgrad_reads_decreasing_ends_as_running_max(gpu, split):
    # with a split the chunk count stays within the workspace the shapes size
    ends = np.array([1024, 0, 1024, 512, 2048], dtype=np.int32)
    M, N, K = 2048, 256, 256
    go, gos = _rand_q((N, M), gpu, 100)
    ia, ias = _rand_q((K, M), gpu, 101)
    dw = ops.grouped_wgrad(go.view(F8), ia.view(F8), torch.from_numpy(ends).to(gpu), gos, ias,
                           out_dtype=torch.float32, split_tokens=split)
    ref = O.grouped_wgrad(u8(go), u8(gos), u8(ia), u8(ias), ends)
    for e, (b, t) in enumerate(O.group_bounds(ends, M)):
        if t > b:
            assert_close_to_oracle(dw[e], ref[e])
        else:
            assert torch.all(dw[e] == 0)


def test_zero_rows_past_groups(gpu):
    out = torch.full((100, 24), 7.0, dtype=torch.bfloat16, device=gpu)
    mxfp8gg.zero_rows_past_groups(out, torch.tensor([10, 60, 30], dtype=torch.int32, device=gpu))
    assert torch.all(out[:60] == 7) and torch.all(out[60:] == 0)
    view = torch.full((50, 40), 3.0, dtype=torch.float32, device=gpu)[:, :32]
    mxfp8gg.zero_rows_past_groups(view, torch.tensor([500], dtype=torch.int32, device=gpu))
    assert torch.all(view == 3)
    mxfp8gg.zero_rows_past_groups(view, torch.tensor([-4], dtype=torch.int32, device=gpu))
    assert torch.all(view == 0)
