"""GPU parity of the MXFP8 data gradient dX = dY . W (blocks along N) through
the C ABI: the weight cast against the oracle bit for bit, the product against
the oracle's dequantise-then-float64 matmul, and against the unquantised
product to MXFP8 accuracy (which a transposed or swapped operand would fail)."""
import numpy as np
import pytest
import torch

import mxfp8gg
from mxfp8gg import workloads
from oracle import oracle as O
from tests._helpers import assert_close_to_oracle, bits, u8

pytestmark = pytest.mark.gpu


def _weights(E, N, K, gpu, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    return (torch.randn(E, N, K, generator=g, device=gpu) * 0.02).to(torch.bfloat16)


@pytest.mark.parametrize("mode_name,mode", [("rceil", O.RCEIL), ("floor", O.FLOOR)])
def test_weight_cast_for_dgrad_is_bit_exact(gpu, mode_name, mode):
    E, N, K = 3, 64, 96
    w = _weights(E, N, K, gpu, 71)
    wt, wts = mxfp8gg.quant_weight_for_dgrad(w, mode_name)
    assert wt.shape == (E, K, N) and wts.shape == (E, K, N // 32)
    ends = (np.arange(1, E + 1) * N).astype(np.int32)
    cap = mxfp8gg.padded_token_capacity(E * N, E)
    rq, rs, rpad = O.quant_dim1(bits(w.reshape(E * N, K)), ends, cap, mode)
    assert np.array_equal(rpad, ends)
    for e in range(E):
        assert np.array_equal(u8(wt[e]), rq[:, e * N:(e + 1) * N])
        assert np.array_equal(u8(wts[e]), rs[:, e * N // 32:(e + 1) * N // 32])


@pytest.mark.parametrize("sizes", [[40, 0, 77, 33], [256], [1, 300, 0]])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_dgrad_matches_oracle(gpu, sizes, out_dtype):
    E, N, K = len(sizes), 96, 160
    M = sum(sizes)
    g = torch.Generator(device=gpu).manual_seed(72)
    dy = (torch.randn(M, N, generator=g, device=gpu) * 1e-2).to(torch.bfloat16)
    w = _weights(E, N, K, gpu, 73)
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    dx = mxfp8gg.grouped_dgrad(dy, w, offs, out_dtype=out_dtype)
    assert dx.shape == (M, K) and dx.dtype == out_dtype
    # oracle: the same casts (pinned separately) then dequantise + float64 matmul
    dyq, dys = mxfp8gg.to_mxfp8_dim0(dy)
    wt, wts = mxfp8gg.quant_weight_for_dgrad(w)
    ref = O.grouped_fwd(u8(dyq), u8(dys), u8(wt), u8(wts), workloads.ends_of(sizes))
    assert_close_to_oracle(dx, ref)
    # the unquantised product dY_g . W_g agrees to MXFP8 accuracy
    full = torch.cat([dy[b:e].float() @ w[i].float()
                      for i, (b, e) in enumerate(O.group_bounds(workloads.ends_of(sizes), M))])
    assert (dx.float() - full).abs().max() / full.abs().max() < 0.1


def test_dgrad_down_projection_shape_sampled_rows(gpu):
    # DSv3 down projection: dY [M, 7168] . W_down[e] [7168, 2048] -> dH [M, 2048]
    sizes = workloads.dirichlet_sizes(8192, 8, seed=3)
    E, N, K = 8, 7168, 2048
    M = int(sizes.sum())
    g = torch.Generator(device=gpu).manual_seed(74)
    dy = (torch.randn(M, N, generator=g, device=gpu) * 1e-3).to(torch.bfloat16)
    w = _weights(E, N, K, gpu, 75)
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    wt = mxfp8gg.quant_weight_for_dgrad(w)
    dx = mxfp8gg.grouped_dgrad(dy, wt, offs)
    rows = np.sort(np.random.default_rng(76).choice(M, 48, replace=False))
    dyq, dys = mxfp8gg.to_mxfp8_dim0(dy)
    ref = O.grouped_fwd(u8(dyq), u8(dys), u8(wt[0]), u8(wt[1]), workloads.ends_of(sizes), rows=rows)
    assert_close_to_oracle(dx[torch.from_numpy(rows).to(gpu)], ref)
