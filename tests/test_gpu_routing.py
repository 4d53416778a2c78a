"""GPU parity of the token routing around the expert GEMMs, through the C ABI.

Dispatch plan, gather and combine are integer / exactly-rounded work: the
plan (perm, src, group ends, counts) and every gathered or combined bf16 row
must equal the CPU oracle bit for bit; the MXFP8 casts of the gathered rows
must equal the casts of the oracle's gathered rows bit for bit.  The score
gradient is an fp32 dot product over H (summation order differs from the
float64 oracle): |got - ref| <= 1e-5 * sum_h |dout * y| + 1e-30.
"""
import numpy as np
import pytest
import torch

import mxfp8gg
from mxfp8gg import _lib, ops, workloads
from oracle import oracle as O
from tests._helpers import bits, from_bits, u8

pytestmark = pytest.mark.gpu


def _idx(gpu, T, K, E, seed, drop=False):
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, E, (T, K), generator=g, dtype=torch.int32)
    if drop and T > 3:
        idx[1, 0] = -1      # dropped slots: negative and past the last expert
        idx[3, K - 1] = E
    return idx.to(gpu)


def _plan_ref(idx, E, pad):
    T, K = idx.shape
    return O.route_plan(idx.cpu().numpy(), E, pad, T * K + E * (pad - 1))


@pytest.mark.parametrize("T,K,E,pad,drop", [
    (1, 1, 1, 1, False), (37, 2, 3, 32, True), (1000, 8, 32, 32, True), (513, 4, 257, 1, False),
    (300, 6, 1024, 128, True), (4096, 1, 8, 32, False), (0, 2, 4, 32, False)])
def test_route_plan_matches_oracle(gpu, T, K, E, pad, drop):
    idx = _idx(gpu, T, K, E, 7 + T, drop)
    plan = mxfp8gg.route_plan(idx, E, pad)
    perm, src, ends, counts = _plan_ref(idx, E, pad)
    assert np.array_equal(plan.perm.cpu().numpy(), perm)
    assert np.array_equal(plan.src.cpu().numpy(), src)
    assert np.array_equal(plan.offs.cpu().numpy(), ends)
    assert np.array_equal(plan.counts.cpu().numpy(), counts)


def test_route_plan_c5_routing(gpu):
    # 16384 tokens x top-8 over 32 experts with Zipf(1.0) preference: the plan
    # of C5's 131072 routed tokens, and torch's own stable argsort order
    idx_np, _ = workloads.c5_routing()
    idx = torch.from_numpy(idx_np).to(gpu)
    plan = mxfp8gg.route_plan(idx, 32, 32)
    perm, src, ends, counts = _plan_ref(idx, 32, 32)
    assert np.array_equal(plan.perm.cpu().numpy(), perm)
    assert np.array_equal(plan.src.cpu().numpy(), src)
    assert np.array_equal(plan.offs.cpu().numpy(), ends)
    order = torch.argsort(idx.reshape(-1).long(), stable=True)
    s = plan.src[plan.src >= 0]
    assert torch.equal(s.long(), order)


@pytest.mark.parametrize("T,K,E,pad,drop", [
    (2500, 8, 32, 32, True),       # 20000 slots: five workgroups, the last partial
    (1200, 7, 1024, 64, True),     # every expert id range across three workgroups
    (4097, 1, 3, 1, False),        # one slot past the first workgroup
    (6000, 2, 1, 32, False)])      # one expert
def test_route_plan_forms_agree(gpu, T, K, E, pad, drop):
    """The many-workgroup plan (what route_plan runs) and the one-workgroup
    entry write the same perm, src, ends and counts, and both equal the oracle."""
    idx = _idx(gpu, T, K, E, 11 + T, drop)
    plan = mxfp8gg.route_plan(idx, E, pad)
    n = T * K
    rows = n + E * (pad - 1)
    perm = torch.full((n,), 7, dtype=torch.int32, device=gpu)
    src = torch.full((rows,), 7, dtype=torch.int32, device=gpu)
    ends = torch.empty(E, dtype=torch.int32, device=gpu)
    counts = torch.empty(E, dtype=torch.int32, device=gpu)
    lib = _lib.load()
    _lib.check(lib.mxgg_route_plan(idx.data_ptr(), T, K, E, pad, rows, perm.data_ptr(),
                                   src.data_ptr(), ends.data_ptr(), counts.data_ptr(),
                                   torch.cuda.current_stream().cuda_stream), "route_plan")
    assert torch.equal(plan.perm, perm) and torch.equal(plan.src, src)
    assert torch.equal(plan.offs, ends) and torch.equal(plan.counts, counts)
    r_perm, r_src, r_ends, r_counts = _plan_ref(idx, E, pad)
    assert np.array_equal(perm.cpu().numpy(), r_perm)
    assert np.array_equal(src.cpu().numpy(), r_src)
    assert np.array_equal(ends.cpu().numpy(), r_ends)
    assert np.array_equal(counts.cpu().numpy(), r_counts)


@pytest.mark.parametrize("scaled", [False, True])
def test_gather_rows_matches_oracle(gpu, scaled):
    T, K, E, H = 301, 3, 5, 96
    idx = _idx(gpu, T, K, E, 3, drop=True)
    g = torch.Generator(device=gpu).manual_seed(4)
    x = torch.randn(T, H, generator=g, device=gpu).to(torch.bfloat16)
    sc = torch.rand(T, K, generator=g, device=gpu) if scaled else None
    plan = mxfp8gg.route_plan(idx, E, 32)
    got = mxfp8gg.gather_rows(x, plan, sc)
    ref = O.gather_rows(bits(x), plan.src.cpu().numpy(), K, sc.cpu().numpy() if scaled else None)
    assert np.array_equal(bits(got), ref)


@pytest.mark.parametrize("mode_name,mode", [("rceil", O.RCEIL), ("floor", O.FLOOR)])
@pytest.mark.parametrize("scaled,pad", [(False, 32), (True, 32), (False, 1)])
def test_gather_to_mxfp8_dual_equals_cast_of_gathered_rows(gpu, mode_name, mode, scaled, pad):
    T, K, E, H = 700, 4, 6, 128
    idx = _idx(gpu, T, K, E, 5, drop=True)
    g = torch.Generator(device=gpu).manual_seed(6)
    x = (torch.randn(T, H, generator=g, device=gpu) * 3).to(torch.bfloat16)
    x[9, 5] = float("nan")
    sc = torch.rand(T, K, generator=g, device=gpu) if scaled else None
    plan = mxfp8gg.route_plan(idx, E, pad)
    q, s, qt, st, offs_pad = mxfp8gg.gather_to_mxfp8_dual(x, plan, mode_name, row_scale=sc)
    xr = mxfp8gg.gather_rows(x, plan, sc)
    q2, s2, qt2, st2, pad2 = mxfp8gg.to_mxfp8_dual(xr, plan.offs, mode_name)
    assert torch.equal(offs_pad, pad2)
    ends = plan.offs.cpu().numpy()
    inside = np.zeros(plan.rows, dtype=bool)
    inside[:ends[-1]] = True   # the row-wise cast writes the rows inside the groups
    assert np.array_equal(u8(q)[inside], u8(q2)[inside])
    assert np.array_equal(u8(s)[inside], u8(s2)[inside])
    assert torch.equal(qt.view(torch.uint8), qt2.view(torch.uint8))
    assert torch.equal(st.contiguous(), st2.contiguous())
    # and the casts themselves against the oracle
    rq, rs = O.quant_dim0(bits(xr)[inside], mode)
    assert np.array_equal(u8(q)[inside], rq) and np.array_equal(u8(s)[inside], rs)
    cap = qt.shape[1]
    rqt, rst, rpad = O.quant_dim1(bits(xr), ends, cap, mode)
    assert np.array_equal(u8(qt), rqt) and np.array_equal(u8(st), rst)


@pytest.mark.parametrize("mode_name,mode", [("rceil", O.RCEIL), ("floor", O.FLOOR)])
@pytest.mark.parametrize("T,K,E,H,pad", [(700, 4, 6, 128, 32), (1, 1, 1, 32, 1),
                                         (333, 10, 40, 7168, 32), (0, 2, 3, 64, 32)])
def test_gather_to_mxfp8_dim0_matches_oracle(gpu, mode_name, mode, T, K, E, H, pad):
    # every routed row (padding rows included) is the row-wise cast of the
    # oracle's gathered row, and equals the cast of the bf16 gathered copy
    idx = _idx(gpu, T, K, E, 14, drop=True)
    g = torch.Generator(device=gpu).manual_seed(15)
    x = (torch.randn(T, H, generator=g, device=gpu) *
         torch.exp2(torch.randint(-30, 30, (T, 1), generator=g, device=gpu).float())
         ).to(torch.bfloat16)
    if T > 9:
        x[9, 5] = float("nan")
        x[2, H - 1] = float("-inf")
    plan = mxfp8gg.route_plan(idx, E, pad)
    q, s = mxfp8gg.gather_to_mxfp8_dim0(x, plan, mode_name)
    assert q.shape == (plan.rows, H) and s.shape == (plan.rows, H // 32)
    xr = O.gather_rows(bits(x), plan.src.cpu().numpy(), K, None)
    rq, rs = O.quant_dim0(xr, mode)
    assert np.array_equal(u8(q), rq) and np.array_equal(u8(s), rs)
    q2, s2 = mxfp8gg.to_mxfp8_dim0(mxfp8gg.gather_rows(x, plan), mode_name)
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8))
    assert torch.equal(s.contiguous(), s2.contiguous())


def test_gather_to_mxfp8_dim0_past_one_grid_pass(gpu):
    # more routed rows than one pass of the gathered cast's grid (2^20 blocks
    # of 32 rows): the rows past it come from the grid-stride loop.  Every
    # routed row must be the cast of its token's row (zero for padding).
    T, K, H = 1000, 4, 32
    rows = (1 << 25) + 96
    g = torch.Generator(device=gpu).manual_seed(19)
    x = torch.randn(T, H, generator=g, device=gpu).to(torch.bfloat16)
    src = torch.randint(-T * K // 8, T * K, (rows,), generator=g, device=gpu, dtype=torch.int32)
    src[src < 0] = -1
    q = torch.zeros((rows, H), dtype=torch.uint8, device=gpu)
    sbuf = ops._block_major_buffer(rows, H // 32, gpu)
    lib = _lib.load()
    st = lib.mxgg_gather_quant_dim0(x.data_ptr(), T, H, H, src.data_ptr(), K, rows, q.data_ptr(), H,
                                    sbuf.data_ptr(), sbuf.stride(0), _lib.SCALES_BLOCK_MAJOR,
                                    _lib.SCALE_RCEIL, torch.cuda.current_stream(gpu).cuda_stream)
    assert st == 0, lib.mxgg_last_error()
    rq, rs = O.quant_dim0(bits(x), O.RCEIL)
    # per token: payload row and scale byte, then gathered on the device
    tq = torch.from_numpy(np.concatenate([rq, np.zeros((1, H), np.uint8)])).to(gpu)
    ts = torch.from_numpy(np.concatenate([rs[:, 0], np.zeros(1, np.uint8)])).to(gpu)
    tok = torch.where(src >= 0, src // K, torch.full_like(src, T)).long()
    assert torch.equal(q, tq[tok])
    assert torch.equal(sbuf[0, :rows], ts[tok])


@pytest.mark.parametrize("scaled", [False, True])
@pytest.mark.parametrize("T,K,E,H", [(257, 8, 32, 64), (40, 1, 3, 24), (1, 2, 2, 8),
                                     (50, 10, 16, 40)])   # top-10: the general slot loop
def test_combine_matches_oracle(gpu, scaled, T, K, E, H):
    idx = _idx(gpu, T, K, E, 8, drop=True)
    plan = mxfp8gg.route_plan(idx, E, 32)
    g = torch.Generator(device=gpu).manual_seed(9)
    y = torch.randn(plan.rows, H, generator=g, device=gpu).to(torch.bfloat16)
    sc = torch.rand(T, K, generator=g, device=gpu) if scaled else None
    got = mxfp8gg.combine(y, plan, sc)
    ref = O.combine(bits(y), plan.perm.cpu().numpy(), K, sc.cpu().numpy() if scaled else None)
    assert np.array_equal(bits(got), ref)


def test_combine_inverts_gather_for_top1(gpu):
    T, E, H = 999, 7, 72
    idx = _idx(gpu, T, 1, E, 10)
    x = torch.randn(T, H, device=gpu).to(torch.bfloat16)
    plan = mxfp8gg.route_plan(idx, E, 32)
    assert torch.equal(mxfp8gg.combine(mxfp8gg.gather_rows(x, plan), plan), x)


@pytest.mark.parametrize("T,K,E,H", [(130, 4, 9, 256), (16, 8, 32, 7168), (33, 11, 12, 64)])
def test_combine_score_grad_matches_oracle(gpu, T, K, E, H):
    idx = _idx(gpu, T, K, E, 11, drop=True)
    plan = mxfp8gg.route_plan(idx, E, 32)
    g = torch.Generator(device=gpu).manual_seed(12)
    y = torch.randn(plan.rows, H, generator=g, device=gpu).to(torch.bfloat16)
    d = torch.randn(T, H, generator=g, device=gpu).to(torch.bfloat16)
    got = mxfp8gg.combine_score_grad(d, y, plan).cpu().numpy().astype(np.float64)
    perm = plan.perm.cpu().numpy()
    ref = O.combine_score_grad(bits(d), bits(y), perm, K)
    mag = O.combine_score_grad(bits(d.abs()), bits(y.abs()), perm, K)
    assert np.all(np.abs(got - ref) <= 1e-5 * mag + 1e-30)
    assert np.all(got[perm.reshape(T, K) < 0] == 0)


# ---------------------------------------------------------------------------
# The routed expert layer
# ---------------------------------------------------------------------------
def _routed_layer(gpu, T=512, K=4, E=8, H=256, F=128, seed=13):
    g = torch.Generator(device=gpu).manual_seed(seed)
    x = torch.randn(T, H, generator=g, device=gpu).to(torch.bfloat16)
    wgu = (torch.randn(E, 2 * F, H, generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    wd = (torch.randn(E, H, F, generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    idx_np, sc_np = workloads.topk_routing(T, E, K, 1.0, seed)
    return x, torch.from_numpy(idx_np).to(gpu), torch.from_numpy(sc_np).to(gpu), wgu, wd


def test_routed_ffn_forward_is_gather_ffn_combine(gpu):
    x, idx, sc, wgu, wd = _routed_layer(gpu)
    E = wgu.shape[0]
    out = mxfp8gg.moe_routed_ffn(x, idx, sc, wgu, wd)
    plan = mxfp8gg.route_plan(idx, E, 32)
    y = mxfp8gg.moe_ffn(mxfp8gg.gather_rows(x, plan), wgu, wd, plan.offs)
    assert torch.equal(out, mxfp8gg.combine(y, plan, sc))


@pytest.mark.parametrize("scored", [True, False])
def test_routed_ffn_forward_only_equals_training_forward(gpu, scored):
    # the no-grad path (row-wise casts only) and the autograd path (dual casts,
    # saved state) give the same bits
    x, idx, sc, wgu, wd = _routed_layer(gpu, T=300, K=6, E=12, seed=16)
    sc = sc if scored else None
    with torch.no_grad():
        a = mxfp8gg.moe_routed_ffn(x, idx, sc, wgu, wd)
    b = mxfp8gg.moe_routed_ffn(x.clone().requires_grad_(True), idx, sc, wgu, wd)
    assert b.requires_grad
    assert torch.equal(a, b.detach())
    cache = mxfp8gg.WeightCastCache()
    with torch.no_grad():
        c = mxfp8gg.moe_routed_ffn(x, idx, sc, wgu, wd, weight_cache=cache)
        d = mxfp8gg.moe_routed_ffn(x, idx, sc, wgu, wd, weight_cache=cache)
    assert torch.equal(a, c) and torch.equal(a, d)


def test_routed_ffn_gradients(gpu):
    # MXFP8 gradients against float32 autograd of the unquantised layer
    # written with torch ops (gather by the stable argsort, per-expert
    # matmuls, score-weighted index_add back to tokens)
    x, idx, sc, wgu, wd = _routed_layer(gpu)
    T, K = idx.shape
    E, F2, H = wgu.shape
    F = F2 // 2
    leaves = [t.clone().requires_grad_(True) for t in (x, sc, wgu, wd)]
    out = mxfp8gg.moe_routed_ffn(leaves[0], idx, leaves[1], leaves[2], leaves[3])
    gout = torch.randn(T, H, device=gpu).to(torch.bfloat16)
    out.backward(gout)

    ref_leaves = [t.detach().float().clone().requires_grad_(True) for t in (x, sc, wgu, wd)]
    xf, scf, wguf, wdf = ref_leaves
    flat = idx.reshape(-1).long()
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=E).tolist()
    xr = xf[order // K]
    outs, lo = [], 0
    for e in range(E):
        hi = lo + counts[e]
        h = xr[lo:hi] @ wguf[e].t()
        outs.append((torch.nn.functional.silu(h[:, :F]) * h[:, F:]) @ wdf[e].t())
        lo = hi
    yr = torch.cat(outs)
    ref = torch.zeros(T, H, device=gpu).index_add_(
        0, order // K, yr * scf.reshape(-1)[order][:, None])
    ref.backward(gout.float())

    def rel(a, b):  # as the unrouted layer's test: max error over max magnitude
        return ((a.float() - b.float()).abs().max() / b.float().abs().max()).item()

    assert rel(out, ref) < 0.1
    for got, want, name in zip(leaves, ref_leaves, ("x", "scores", "w_gate_up", "w_down")):
        assert rel(got.grad, want.grad) < 0.15, name
