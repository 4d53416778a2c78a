"""GPU parity of the expert-FFN layer step (mxfp8gg.moe_ffn, forward and
backward through autograd) against the composed oracle of tests/_layer_oracle:
every GEMM output held against dequantise + float64 matmul at the 1e-2 bound,
every cast bit for bit, SwiGLU forward and backward recomputed by the oracle.

Sizes: toy layers with every row and feature checked (empty experts, group
starts off multiples of 4 and of 32), and BASELINE.json configs[4] (C5) at its
full size -- 131072 tokens routed Zipf(1.0) over 32 experts, hidden 7168,
intermediate 2048 (the reference's layer step, e2e_bench.py:56-134) -- on
sampled rows of y and dX and sampled weight-gradient entries of every expert."""
import numpy as np
import pytest
import torch

import mxfp8gg
from mxfp8gg import workloads
from tests._layer_oracle import check_layer

pytestmark = pytest.mark.gpu


def _layer(gpu, sizes, H, F, seed, wscale=0.006, dyscale=1e-3):
    E, M = len(sizes), int(np.sum(sizes))
    g = torch.Generator(device=gpu).manual_seed(seed)
    x = torch.randn(M, H, generator=g, device=gpu).to(torch.bfloat16)
    wgu = (torch.randn(E, 2 * F, H, generator=g, device=gpu) * wscale).to(torch.bfloat16)
    wd = (torch.randn(E, H, F, generator=g, device=gpu) * wscale).to(torch.bfloat16)
    dy = (torch.randn(M, H, generator=g, device=gpu) * dyscale).to(torch.bfloat16)
    return x, wgu, wd, dy


def _run(x, wgu, wd, dy, sizes):
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(x.device)
    leaves = [t.clone().requires_grad_(True) for t in (x, wgu, wd)]
    y = mxfp8gg.moe_ffn(*leaves, offs)
    y.backward(dy)
    return {"y": y.detach(), "dx": leaves[0].grad, "dwgu": leaves[1].grad, "dwd": leaves[2].grad}


@pytest.mark.parametrize("sizes,H,F", [
    ([64, 128, 0, 96], 256, 128),          # an empty expert, 32-aligned groups
    ([33, 7, 0, 250, 66], 320, 96),        # group starts off multiples of 4 and 32
    ([512], 192, 64),                      # one expert
])
def test_moe_ffn_matches_composed_oracle(gpu, sizes, H, F):
    x, wgu, wd, dy = _layer(gpu, sizes, H, F, 83, wscale=0.06, dyscale=1.0)
    got = _run(x, wgu, wd, dy, sizes)
    M = int(np.sum(sizes))
    check_layer(x, wgu, wd, dy, sizes, np.arange(M), np.arange(H), np.arange(F),
                np.arange(2 * F), np.arange(H), got)


def test_moe_ffn_c5_matches_composed_oracle(gpu):
    sizes = workloads.c5_sizes()
    E, H, F = 32, 7168, 2048
    M = int(sizes.sum())
    assert M == 131072 and sizes.max() > 30000
    print(f"C5 layer step: {M} tokens, sizes min {sizes.min()} max {sizes.max()}", flush=True)
    x, wgu, wd, dy = _layer(gpu, sizes, H, F, 0)
    got = _run(x, wgu, wd, dy, sizes)
    ends = workloads.ends_of(sizes)
    starts = ends - sizes
    rng = np.random.default_rng(5)
    rows = []
    for e in (0, 1, 7, 16, 30, 31):                       # largest .. smallest experts
        b, t = int(starts[e]), int(ends[e])
        rows += [b, t - 1] + rng.integers(b, t, 4).tolist()
    rows = np.unique(np.array(rows))
    n_feat = np.unique(np.r_[0, 2047, 7167, rng.integers(0, H, 5)])
    f_feat = np.unique(np.r_[0, 2047, rng.integers(0, F, 6)])
    m_feat = np.unique(np.r_[0, F - 1, F, 2 * F - 1, rng.integers(0, 2 * F, 4)])
    k_feat = np.unique(np.r_[0, 7167, rng.integers(0, H, 6)])
    check_layer(x, wgu, wd, dy, sizes, rows, n_feat, f_feat, m_feat, k_feat, got)


def test_moe_ffn_past_2gib_matches_composed_oracle(gpu):
    # 300000 tokens x hidden 7168: X, its casts, dY and the token-axis
    # operands of both weight gradients are past the 2 GiB buffer range of one
    # launch, so the forward and dgrad run in row chunks and both weight
    # gradients in feature-row chunks (dY^T of the down projection along its
    # rows, X^T of the gate+up projection along its rows).
    sizes = np.array([120000, 0, 150000, 30000])
    E, H, F = 4, 7168, 2048
    M = int(sizes.sum())
    assert mxfp8gg.padded_token_capacity(M, E) * H > 2 ** 31
    print(f"layer step past 2 GiB: {M} tokens, E={E}", flush=True)
    x, wgu, wd, dy = _layer(gpu, sizes, H, F, 91)
    got = _run(x, wgu, wd, dy, sizes)
    ends = workloads.ends_of(sizes)
    starts = ends - sizes
    rng = np.random.default_rng(9)
    rows = []
    for e in (0, 2, 3):
        b, t = int(starts[e]), int(ends[e])
        rows += [b, t - 1] + rng.integers(b, t, 3).tolist()
    rows = np.unique(np.array(rows))
    n_feat = np.unique(np.r_[0, 6911, 6912, 7167, rng.integers(0, H, 3)])
    f_feat = np.unique(np.r_[0, 2047, rng.integers(0, F, 4)])
    m_feat = np.unique(np.r_[0, F - 1, F, 2 * F - 1, rng.integers(0, 2 * F, 3)])
    k_feat = np.unique(np.r_[0, 6911, 6912, 7167, rng.integers(0, H, 3)])
    check_layer(x, wgu, wd, dy, sizes, rows, n_feat, f_feat, m_feat, k_feat, got)


def test_layer_rows_past_the_groups_are_zero(gpu):
    # offs[-1] < M: rows past the last group end get zero output and zero dX
    sizes = [64, 96, 32]
    E, H, F = 3, 256, 64
    x, wgu, wd, dy = _layer(gpu, sizes + [40], H, F, 87, wscale=0.06, dyscale=1.0)
    wgu, wd = wgu[:E].contiguous(), wd[:E].contiguous()
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    M = x.shape[0]
    end = int(np.sum(sizes))
    leaves = [t.clone().requires_grad_(True) for t in (x, wgu, wd)]
    y = mxfp8gg.moe_ffn(*leaves, offs)
    y.backward(dy)
    assert torch.all(y[end:] == 0) and torch.all(leaves[0].grad[end:] == 0)
    with torch.no_grad():
        assert torch.all(mxfp8gg.moe_ffn(x, wgu, wd, offs)[end:] == 0)
    xa = x.clone().requires_grad_(True)
    w1 = wgu.clone().requires_grad_(True)
    y1 = mxfp8gg.mxfp8_grouped_mm(xa, w1, offs)
    y1.backward(torch.ones_like(y1))
    assert torch.all(y1[end:] == 0) and torch.all(xa.grad[end:] == 0)
    assert torch.isfinite(xa.grad).all() and M > end
    # the rows inside the groups agree with the layer computed on them alone
    got = _run(x[:end], wgu, wd, dy[:end], sizes)
    assert torch.equal(y[:end], got["y"])
    assert torch.equal(leaves[0].grad[:end], got["dx"])
