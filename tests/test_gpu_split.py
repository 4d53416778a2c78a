"""GPU parity of the forward's split last round (mxgg_grouped_fwd_split).

When the tiles of the last round would leave at least half of the compute
units idle, they run cut along K over the idle units, and a second kernel adds
the fp32 partials in a fixed order.  The tests call the C ABI with their own
workspace so that the header the kernel writes (number of split tiles, split
count) shows the split happened, and check:

  * against the float64 dequantise-then-matmul oracle, with the GEMM tolerance
    of every other forward test (tests/_helpers.assert_close_to_oracle);
  * against the unsplit entry point: equal up to fp32 summation order
    (|split - unsplit| <= 2^-14 * max|unsplit| for fp32 output: every MFMA
    adds into a different running sum; one bf16 unit in the last place of the
    largest value for bf16 output);
  * bit-for-bit determinism of repeated calls, and bit-equal results where
    every partial sum is exact (power-of-two products).
"""
import numpy as np
import pytest
import torch

from mxfp8gg import _lib, ops
from oracle import oracle as O
from tests._helpers import assert_close_to_oracle, u8

pytestmark = pytest.mark.gpu

F8 = torch.float8_e4m3fn


def _grid(gpu):
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    return (cus + 7) // 8 * 8


def _rand_q(shape, gpu, seed, lo=118, hi=136):
    g = torch.Generator(device=gpu).manual_seed(seed)
    codes = torch.randint(0, 0x7E, shape, generator=g, device=gpu, dtype=torch.int32)
    sign = torch.randint(0, 2, shape, generator=g, device=gpu, dtype=torch.int32) << 7
    s = torch.randint(lo, hi, shape[:-1] + (shape[-1] // 32,), generator=g, device=gpu,
                      dtype=torch.int32).to(torch.uint8)
    return (codes | sign).to(torch.uint8).view(F8), s


def _fwd(gpu, a, w, ends, a_s, w_s, out_dtype, split):
    """One forward through the C ABI; returns (out, header ints or None)."""
    M, K = a.shape
    E, N, _ = w.shape
    sa, ldas = ops._scales_2d(a_s, M, K // 32, "a_s") if a_s is not None else (None, 0)
    sw, wsg, ldws = ops._scales_3d(w_s, E, N, K // 32, "w_s") if w_s is not None else (None, 0, 0)
    out = torch.full((M, N), float("nan"), dtype=out_dtype, device=gpu)
    lib = _lib.load()
    a8, w8 = a.view(torch.uint8), w.view(torch.uint8)
    args = (a8.data_ptr(), a8.stride(0), sa.data_ptr() if sa is not None else None, ldas,
            w8.data_ptr(), w8.stride(0), w8.stride(1), sw.data_ptr() if sw is not None else None,
            wsg, ldws, ends.data_ptr() if ends is not None else None, E, M, N, K, out.data_ptr(),
            out.stride(0), ops._out_code(out_dtype))
    stream = torch.cuda.current_stream(gpu).cuda_stream
    if not split:
        _lib.check(lib.mxgg_grouped_fwd(*args, stream), "grouped_fwd")
        return out, None
    nbytes = lib.mxgg_grouped_fwd_workspace_bytes()
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    _lib.check(lib.mxgg_grouped_fwd_split(*args, ws.data_ptr(), nbytes, stream), "grouped_fwd_split")
    torch.cuda.synchronize()
    return out, ws[:8].view(torch.int32).cpu().tolist()


def _expect_split(G, tiles, K):
    """(split tiles, split count) the kernel should choose."""
    rem = tiles % G
    nst = (K + 127) // 128
    if rem == 0 or rem > G // 2 or nst < 2:
        return 0
    S = min(G // rem, nst, 16 if tiles < G else 8)
    chunk = -(-nst // S)
    return rem, -(-nst // chunk)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_sparse_last_round_is_split_and_matches(gpu, out_dtype):
    # one expert, 17 x 16 tiles: a last round of 16 tiles on a 256-unit device
    G = _grid(gpu)
    M, N, K = 256 * 17, 256 * 16, 2048
    a, a_s = _rand_q((M, K), gpu, 1)
    w, w_s = _rand_q((1, N, K), gpu, 2)
    y, hdr = _fwd(gpu, a, w, None, a_s, w_s, out_dtype, True)
    exp = _expect_split(G, 17 * 16, K)
    if exp:
        assert tuple(hdr[:2]) == exp
    y0, _ = _fwd(gpu, a, w, None, a_s, w_s, out_dtype, False)
    diff = (y.float() - y0.float()).abs().max().item()
    mag = y0.float().abs().max().item()
    if out_dtype == torch.float32:
        assert diff <= 2.0 ** -14 * mag
    else:   # one bf16 rounding step of the largest value at most
        assert diff <= 2.0 ** -7 * mag
    # the rows of the last round against the oracle (tile order puts them last)
    rows = np.r_[0:64, M - 300:M]
    ref = O.grouped_fwd(u8(a)[rows], u8(a_s)[rows], u8(w), u8(w_s), np.array([rows.size]))
    assert_close_to_oracle(y[torch.from_numpy(rows).to(gpu)], ref)
    y2, _ = _fwd(gpu, a, w, None, a_s, w_s, out_dtype, True)
    assert torch.equal(y.view(torch.int8) if out_dtype == torch.bfloat16 else y,
                       y2.view(torch.int8) if out_dtype == torch.bfloat16 else y2)


@pytest.mark.parametrize("sizes,N,K,scaled", [
    ([200], 200, 7168, True),                 # one tile, 56 stages: 16 ranges of 4 stages
    ([37, 0, 300, 5, 129], 96, 384, True),    # ragged groups, 3 stages
    ([3, 29, 45, 1], 40, 4096, False),        # unscaled
    ([513], 264, 128, True),                  # a single stage: no split
])
def test_small_launch_split_matches_oracle(gpu, sizes, N, K, scaled):
    G = _grid(gpu)
    M, E = sum(sizes), len(sizes)
    a, a_s = _rand_q((M, K), gpu, 3)
    w, w_s = _rand_q((E, N, K), gpu, 4)
    ends = torch.tensor(np.cumsum(sizes), dtype=torch.int32, device=gpu)
    a_s, w_s = (a_s, w_s) if scaled else (None, None)
    y, hdr = _fwd(gpu, a, w, ends, a_s, w_s, torch.float32, True)
    starts = np.r_[0, np.cumsum(sizes)[:-1]]
    tiles = sum(-(-(e - (b & ~3)) // 256) for b, e in zip(starts, np.cumsum(sizes)) if e > b)
    tiles *= -(-N // 256)
    exp = _expect_split(G, tiles, K)
    assert tuple(hdr[:2]) == (exp if exp else (0, 1))
    ref = O.grouped_fwd(u8(a), u8(a_s) if scaled else None, u8(w), u8(w_s) if scaled else None,
                        np.cumsum(sizes))
    assert_close_to_oracle(y, ref)
    y0, _ = _fwd(gpu, a, w, ends, a_s, w_s, torch.float32, False)
    assert (y - y0).abs().max().item() <= 2.0 ** -14 * y0.abs().max().item()


def test_split_sums_are_exact_for_exact_partials(gpu):
    # every product is a power of two and every partial sum is exact in fp32,
    # so the split result equals the unsplit one bit for bit; one column has
    # only -0 products (a sum that starts from +0 is +0 on both paths)
    M, N, K = 64, 64, 4096
    a = torch.full((M, K), 0x38, dtype=torch.uint8, device=gpu)           # 1.0
    w = torch.full((1, N, K), 0x38, dtype=torch.uint8, device=gpu)
    w[0, 7] = 0x80                                                         # -0
    a_s = torch.full((M, K // 32), 127, dtype=torch.uint8, device=gpu)
    a_s[:, ::3] = 128
    w_s = torch.full((1, N, K // 32), 127, dtype=torch.uint8, device=gpu)
    y, hdr = _fwd(gpu, a.view(F8), w.view(F8), None, a_s, w_s, torch.float32, True)
    assert hdr[0] == 1 and hdr[1] > 1
    y0, _ = _fwd(gpu, a.view(F8), w.view(F8), None, a_s, w_s, torch.float32, False)
    assert torch.equal(y.view(torch.int32), y0.view(torch.int32))
    assert torch.all(y[:, 7] == 0)
    expect = 32.0 * ((K // 32 + 2) // 3 * 2 + (K // 32 - (K // 32 + 2) // 3))
    assert torch.all(y[:, :7] == expect)


def test_split_workspace_is_validated(gpu):
    lib = _lib.load()
    n = lib.mxgg_grouped_fwd_workspace_bytes()
    assert n >= 16384 + _grid(gpu) * 256 * 256 * 4
    a = torch.zeros((32, 64), dtype=torch.uint8, device=gpu)
    w = torch.zeros((1, 32, 64), dtype=torch.uint8, device=gpu)
    out = torch.empty((32, 32), dtype=torch.bfloat16, device=gpu)
    ws = torch.empty(n, dtype=torch.uint8, device=gpu)
    args = (a.data_ptr(), 64, None, 0, w.data_ptr(), 32 * 64, 64, None, 0, 0, None, 1, 32, 32, 64,
            out.data_ptr(), 32, _lib.OUT_BF16)
    assert lib.mxgg_grouped_fwd_split(*args, ws.data_ptr(), n - 1, None) == _lib.ERR_SHAPE
    assert lib.mxgg_grouped_fwd_split(*args, None, n, None) == _lib.ERR_INVALID_ARGUMENT
    assert lib.mxgg_grouped_fwd_split(*args, ws.data_ptr() + 4, n, None) == _lib.ERR_ALIGNMENT
    assert lib.mxgg_grouped_fwd_split(*args, ws.data_ptr(), n, None) == _lib.OK
    torch.cuda.synchronize()
    assert torch.all(out == 0)
