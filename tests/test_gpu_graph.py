"""HIP graph capture of the library's launches (torch.cuda.CUDAGraph).

Small calls are launch-bound, so callers capture them.  Every entry point
launches on the current stream, allocates nothing in the library (outputs and
workspaces come from torch's allocator, the graph's pool during capture) and
records no memset (the split kernels write their own headers).  The test
captures a routed step and a split weight gradient once, then replays the graph
several times with new inputs written in place by eager work between replays,
and checks every replay bit for bit against the same calls run eagerly.
"""
import pytest
import torch

import mxfp8gg
from mxfp8gg import ops, workloads

pytestmark = pytest.mark.gpu


def _fill(gen, *ts):
    for t in ts:
        t.copy_(torch.randn(t.shape, generator=gen, device=t.device) * 0.5)


def test_graph_replays_match_eager(gpu):
    T, K, E, H, F = 96, 4, 8, 256, 128          # 384 routed slots, small launches
    gen = torch.Generator(device=gpu).manual_seed(71)
    x = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
    wgu = torch.empty((E, 2 * F, H), dtype=torch.bfloat16, device=gpu)
    wd = torch.empty((E, H, F), dtype=torch.bfloat16, device=gpu)
    dy = torch.empty((E * 512, H), dtype=torch.bfloat16, device=gpu)
    xw = torch.empty((E * 512, 2 * F), dtype=torch.bfloat16, device=gpu)
    idx_np, sc_np = workloads.topk_routing(T, E, K, 1.0, 71)
    idx = torch.from_numpy(idx_np).to(gpu)
    sc = torch.from_numpy(sc_np).to(gpu)
    ends = torch.arange(1, E + 1, dtype=torch.int32, device=gpu) * 512
    _fill(gen, x, wgu, wd, dy, xw)

    def step():
        plan = mxfp8gg.route_plan(idx, E)
        q, s, _, _, _ = mxfp8gg.gather_to_mxfp8_dual(x, plan)
        (wq, ws), _ = ops.quant_weight_dual(wgu)
        h = ops.grouped_mm(q, wq, plan.offs, s, ws)                 # split launch
        aq, as_ = ops.swiglu_quant(h)
        (dq, ds), _ = ops.quant_weight_dual(wd)
        y = ops.grouped_mm(aq, dq, plan.offs, as_, ds)
        out = mxfp8gg.combine(y, plan, sc)
        go, gos, pad = mxfp8gg.to_mxfp8_dim1(dy, ends)
        ia, ias, _ = mxfp8gg.to_mxfp8_dim1(xw, ends)
        dw = ops.grouped_wgrad(go, ia, pad, gos, ias, out_dtype=torch.bfloat16,
                               split_tokens=256)                   # staged split
        return out, dw

    # warm up on a side stream (library load, size queries, allocator pools)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_out, g_dw = step()
    for _ in range(3):
        _fill(gen, x, wgu, wd, dy, xw)                 # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        e_out, e_dw = step()
        torch.cuda.synchronize()
        assert torch.equal(g_out.view(torch.int16), e_out.view(torch.int16))
        assert torch.equal(g_dw.view(torch.int16), e_dw.view(torch.int16))
        assert torch.isfinite(e_out.float()).all()


def test_graph_of_routed_forward_only(gpu):
    # the whole forward-only routed layer captured as one graph
    # (plan, gathered cast, weight casts, two GEMMs, SwiGLU cast, combine)
    T, K, E, H, F = 64, 8, 16, 256, 128
    gen = torch.Generator(device=gpu).manual_seed(72)
    x = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
    wgu = torch.empty((E, 2 * F, H), dtype=torch.bfloat16, device=gpu)
    wd = torch.empty((E, H, F), dtype=torch.bfloat16, device=gpu)
    _fill(gen, x, wgu, wd)
    idx_np, sc_np = workloads.topk_routing(T, E, K, 1.0, 72)
    idx = torch.from_numpy(idx_np).to(gpu)
    sc = torch.from_numpy(sc_np).to(gpu)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mxfp8gg.moe_routed_ffn(x, idx, sc, wgu, wd)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_out = mxfp8gg.moe_routed_ffn(x, idx, sc, wgu, wd)
    for r in range(3):
        _fill(gen, x)
        i2, s2 = workloads.topk_routing(T, E, K, 1.0, 100 + r)
        idx.copy_(torch.from_numpy(i2).to(gpu))
        sc.copy_(torch.from_numpy(s2).to(gpu))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        e_out = mxfp8gg.moe_routed_ffn(x, idx, sc, wgu, wd)
        torch.cuda.synchronize()
        assert torch.equal(g_out.view(torch.int16), e_out.view(torch.int16))


def test_graph_replays_route_plan_over_workgroups(gpu):
    """The routing plan past 4096 slots (count, offsets and rank kernels with a
    workspace from the graph's pool) captured once and replayed with new
    expert ids written in place: every replay equals the eager plan."""
    T, K, E = 1536, 8, 32                        # 12288 slots: three workgroups
    gen = torch.Generator(device=gpu).manual_seed(5)
    idx = torch.empty((T, K), dtype=torch.int32, device=gpu)

    def new_idx():
        idx.copy_(torch.randint(0, E, (T, K), generator=gen, device=gpu, dtype=torch.int32))

    new_idx()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mxfp8gg.route_plan(idx, E)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g = mxfp8gg.route_plan(idx, E)
    for _ in range(3):
        new_idx()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        e = mxfp8gg.route_plan(idx, E)
        torch.cuda.synchronize()
        for a, b in zip((g.perm, g.src, g.offs, g.counts), (e.perm, e.src, e.offs, e.counts)):
            assert torch.equal(a, b)
