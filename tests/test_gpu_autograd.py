"""GPU tests of the differentiable MXFP8 grouped GEMM (forward, dgrad and
wgrad through the C ABI): identical to the explicit ops it is built from, and
gradients equal to float32 autograd of the unquantised math to MXFP8
accuracy, which pins the operand orientation of every product."""
import numpy as np
import pytest
import torch

import mxfp8gg
from mxfp8gg import ops, workloads

pytestmark = pytest.mark.gpu


def _inputs(gpu, sizes, N, K, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    M = sum(sizes)
    x = torch.randn(M, K, generator=g, device=gpu).to(torch.bfloat16)
    w = (torch.randn(len(sizes), N, K, generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    dy = (torch.randn(M, N, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    return x, w, dy, offs


def _rel(a, b):
    return ((a.float() - b.float()).abs().max() / b.float().abs().max()).item()


@pytest.mark.parametrize("sizes", [[64, 0, 96, 32], [200]])
def test_autograd_equals_explicit_ops(gpu, sizes):
    x, w, dy, offs = _inputs(gpu, sizes, 128, 160, 81)
    xa = x.clone().requires_grad_(True)
    wa = w.clone().requires_grad_(True)
    y = mxfp8gg.mxfp8_grouped_mm(xa, wa, offs)
    y.backward(dy)
    xq, xs = ops.to_mxfp8_dim0(x)
    wq, ws = ops.to_mxfp8_dim0(w)
    assert torch.equal(y, ops.grouped_mm(xq, wq, offs, xs, ws))
    assert torch.equal(xa.grad, ops.grouped_dgrad(dy, w, offs))
    go, gos, pad = ops.to_mxfp8_dim1(dy, offs)
    ia, ias, _ = ops.to_mxfp8_dim1(x, offs)
    assert torch.equal(wa.grad, ops.grouped_wgrad(go, ia, pad, gos, ias, out_dtype=torch.bfloat16))


@pytest.mark.parametrize("sizes", [[96, 0, 160, 64], [33, 7, 250]])
def test_autograd_gradients_match_fp32(gpu, sizes):
    x, w, dy, offs = _inputs(gpu, sizes, 192, 256, 82)
    xa = x.clone().requires_grad_(True)
    wa = w.clone().requires_grad_(True)
    mxfp8gg.mxfp8_grouped_mm(xa, wa, offs).backward(dy)
    xr = x.float().requires_grad_(True)
    wr = w.float().requires_grad_(True)
    ends = workloads.ends_of(sizes)
    yr = torch.cat([xr[b:e] @ wr[g].T for g, (b, e) in
                    enumerate(zip(np.r_[0, ends[:-1]], ends))])
    yr.backward(dy.float())
    assert _rel(xa.grad, xr.grad) < 0.1
    assert _rel(wa.grad, wr.grad) < 0.1
    for g, s in enumerate(sizes):
        if s == 0:
            assert torch.all(wa.grad[g] == 0)


def test_moe_ffn_layer_gradients_match_fp32(gpu):
    sizes = [64, 128, 0, 96]
    E, H, F = 4, 256, 128
    g = torch.Generator(device=gpu).manual_seed(83)
    M = sum(sizes)
    x = torch.randn(M, H, generator=g, device=gpu).to(torch.bfloat16)
    wgu = (torch.randn(E, 2 * F, H, generator=g, device=gpu) * 0.06).to(torch.bfloat16)
    wd = (torch.randn(E, H, F, generator=g, device=gpu) * 0.06).to(torch.bfloat16)
    dy = torch.randn(M, H, generator=g, device=gpu).to(torch.bfloat16)
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    leaves = [t.clone().requires_grad_(True) for t in (x, wgu, wd)]
    y = mxfp8gg.moe_ffn(*leaves, offs)
    y.backward(dy)
    ref = [t.float().requires_grad_(True) for t in (x, wgu, wd)]
    ends = workloads.ends_of(sizes)
    outs = []
    for e, (b, t) in enumerate(zip(np.r_[0, ends[:-1]], ends)):
        h = ref[0][b:t] @ ref[1][e].T
        a = torch.nn.functional.silu(h[:, :F]) * h[:, F:]
        outs.append(a @ ref[2][e].T)
    yr = torch.cat(outs)
    yr.backward(dy.float())
    assert _rel(y, yr) < 0.1
    for got, want in zip(leaves, ref):
        assert _rel(got.grad, want.grad) < 0.15


def test_moe_ffn_fused_matches_unfused_composition(gpu):
    # The fused layer (SwiGLU kernels) against the composition of two
    # MXFP8GroupedMM calls with torch's eager bf16 SiLU * up.
    sizes = [64, 160, 0, 96, 32]
    E, H, F = 5, 256, 192
    g = torch.Generator(device=gpu).manual_seed(84)
    M = sum(sizes)
    x = torch.randn(M, H, generator=g, device=gpu).to(torch.bfloat16)
    wgu = (torch.randn(E, 2 * F, H, generator=g, device=gpu) * 0.06).to(torch.bfloat16)
    wd = (torch.randn(E, H, F, generator=g, device=gpu) * 0.06).to(torch.bfloat16)
    dy = torch.randn(M, H, generator=g, device=gpu).to(torch.bfloat16)
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    fused = [t.clone().requires_grad_(True) for t in (x, wgu, wd)]
    plain = [t.clone().requires_grad_(True) for t in (x, wgu, wd)]
    y1 = mxfp8gg.moe_ffn(*fused, offs)
    y1.backward(dy)
    y2 = mxfp8gg.moe_ffn_unfused(*plain, offs)
    y2.backward(dy)
    for got, want in [(y1, y2)] + [(a.grad, b.grad) for a, b in zip(fused, plain)]:
        assert got.shape == want.shape
        assert _rel(got, want) < 1e-2
        assert (got == want).float().mean().item() > 0.99


def test_moe_ffn_weight_cache(gpu):
    sizes = [64, 96, 32]
    E, H, F = 3, 256, 128
    g = torch.Generator(device=gpu).manual_seed(85)
    M = sum(sizes)
    x = torch.randn(M, H, generator=g, device=gpu).to(torch.bfloat16)
    wgu = (torch.randn(E, 2 * F, H, generator=g, device=gpu) * 0.06).to(torch.bfloat16)
    wd = (torch.randn(E, H, F, generator=g, device=gpu) * 0.06).to(torch.bfloat16)
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    cache = mxfp8gg.WeightCastCache()
    ref = mxfp8gg.moe_ffn(x, wgu, wd, offs)
    for _ in range(2):                             # second call reuses both weight casts
        assert torch.equal(mxfp8gg.moe_ffn(x, wgu, wd, offs, weight_cache=cache), ref)
    assert cache.misses == 2 and cache.hits == 2
    with torch.no_grad():
        wd.mul_(0.5)                               # an optimizer-style in-place update
    upd = mxfp8gg.moe_ffn(x, wgu, wd, offs)
    assert torch.equal(mxfp8gg.moe_ffn(x, wgu, wd, offs, weight_cache=cache), upd)
    assert cache.misses == 3
    # with autograd: gradients identical with and without the cache
    leaves = [t.clone().requires_grad_(True) for t in (x, wgu, wd)]
    mxfp8gg.moe_ffn(*leaves, offs).backward(ref)
    leaves_c = [t.clone().requires_grad_(True) for t in (x, wgu, wd)]
    mxfp8gg.moe_ffn(*leaves_c, offs, weight_cache=cache).backward(ref)
    for a, b in zip(leaves, leaves_c):
        assert torch.equal(a.grad, b.grad)
