"""Randomised GPU parity sweep: shapes, group layouts and options drawn from a
seeded generator (each case prints its parameters in its id, so a failure
names and reproduces its case), checked against the CPU oracle with the same
bars as the fixed-case tests:

  * casts, routing plans, gathers and combines: bit for bit;
  * the gate+up GEMM with SwiGLU and the cast in its epilogue (with and
    without the bf16 projection kept): bit for bit against the grouped GEMM
    followed by the standalone SwiGLU cast;
  * grouped GEMMs: tests/_helpers.assert_close_to_oracle (every element within
    2^-7 |ref| + 2^-12 max|ref| of the float64 dequantise-then-matmul value);
    split forwards also within 2^-14 max|y| (fp32) or 2^-7 max|y| (bf16) of
    the unsplit entry point.

Shapes stay small enough for the numpy oracle (a few seconds for the file).
"""
import numpy as np
import pytest
import torch

import mxfp8gg
from mxfp8gg import ops, workloads
from oracle import oracle as O
from tests._helpers import assert_close_to_oracle, bits, u8

pytestmark = pytest.mark.gpu


def _sizes(rng, E, M, zeros=True, mult=1):
    w = rng.dirichlet(np.ones(E))
    sizes = rng.multinomial(M // mult, w) * mult
    if zeros and E > 2:
        sizes[rng.integers(0, E)] = 0
    return [int(s) for s in sizes]


def _fwd_cases(n=16, seed=100):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        E = int(rng.integers(1, 24))
        M = int(rng.integers(1, 600))
        out.append((_sizes(rng, E, M), 16 * int(rng.integers(1, 26)), 32 * int(rng.integers(1, 17)),
                    bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), int(rng.integers(0, 2**31))))
    return out


def _rand_q(shape, gpu, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    codes = torch.randint(0, 0x7E, shape, generator=g, device=gpu, dtype=torch.int32)
    sign = torch.randint(0, 2, shape, generator=g, device=gpu, dtype=torch.int32) << 7
    s = torch.randint(118, 136, shape[:-1] + (shape[-1] // 32,), generator=g, device=gpu,
                      dtype=torch.int32).to(torch.uint8)
    return (codes | sign).to(torch.uint8), s


@pytest.mark.parametrize("sizes,N,K,scaled,f32,seed", _fwd_cases())
def test_random_grouped_fwd(gpu, sizes, N, K, scaled, f32, seed):
    E, M = len(sizes), sum(sizes)
    a_q, a_s = _rand_q((max(M, 1), K), gpu, seed)
    w_q, w_s = _rand_q((E, N, K), gpu, seed + 1)
    a_q, a_s = a_q[:M], a_s[:M]
    ends = workloads.ends_of(sizes)
    y = ops.grouped_mm(a_q.view(torch.float8_e4m3fn), w_q.view(torch.float8_e4m3fn),
                       torch.from_numpy(ends).to(gpu), a_s if scaled else None,
                       w_s if scaled else None,
                       out_dtype=torch.float32 if f32 else torch.bfloat16)
    if M == 0:
        return
    ref = O.grouped_fwd(u8(a_q), u8(a_s) if scaled else None, u8(w_q),
                        u8(w_s) if scaled else None, ends)
    assert_close_to_oracle(y, ref)


def _split_cases(n=12, seed=150):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        E = int(rng.integers(1, 9))
        M = int(rng.integers(1, 1500))
        out.append((_sizes(rng, E, M), 8 * int(rng.integers(1, 76)), 32 * int(rng.integers(1, 129)),
                    bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), int(rng.integers(0, 2**31))))
    return out


@pytest.mark.parametrize("sizes,N,K,scaled,f32,seed", _split_cases())
def test_random_split_forward(gpu, sizes, N, K, scaled, f32, seed):
    # small launches split along K (mxgg_grouped_fwd_split) against the oracle
    # and against the unsplit entry point (fp32 summation order only)
    E, M = len(sizes), sum(sizes)
    a_q, a_s = _rand_q((max(M, 1), K), gpu, seed)
    w_q, w_s = _rand_q((E, N, K), gpu, seed + 1)
    a_q, a_s = a_q[:M], a_s[:M]
    ends = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    dt = torch.float32 if f32 else torch.bfloat16
    args = (a_q.view(torch.float8_e4m3fn), w_q.view(torch.float8_e4m3fn), ends,
            a_s if scaled else None, w_s if scaled else None)
    y1 = ops.grouped_mm(*args, out_dtype=dt, split_tail=True)
    y0 = ops.grouped_mm(*args, out_dtype=dt, split_tail=False)
    if M == 0:
        return
    ref = O.grouped_fwd(u8(a_q), u8(a_s) if scaled else None, u8(w_q),
                        u8(w_s) if scaled else None, workloads.ends_of(sizes))
    assert_close_to_oracle(y1, ref)
    mag = y0.float().abs().max().item()
    assert (y1.float() - y0.float()).abs().max().item() <= (2.0 ** -14 if f32 else 2.0 ** -7) * mag


def _wgrad_cases(n=10, seed=200):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        E = int(rng.integers(1, 8))
        M = 32 * int(rng.integers(1, 40))
        f32 = bool(rng.integers(0, 2))
        split = 128 * int(rng.integers(1, 4)) if f32 and rng.integers(0, 2) else 0
        out.append((_sizes(rng, E, M, mult=32), 16 * int(rng.integers(1, 24)),
                    16 * int(rng.integers(1, 24)), f32, split, int(rng.integers(0, 2**31))))
    return out


@pytest.mark.parametrize("sizes,N,K,f32,split,seed", _wgrad_cases())
def test_random_grouped_wgrad(gpu, sizes, N, K, f32, split, seed):
    M = sum(sizes)
    go_q, go_s = _rand_q((N, M), gpu, seed)
    ia_q, ia_s = _rand_q((K, M), gpu, seed + 1)
    ends = workloads.ends_of(sizes)
    dw = ops.grouped_wgrad(go_q.view(torch.float8_e4m3fn), ia_q.view(torch.float8_e4m3fn),
                           torch.from_numpy(ends).to(gpu), go_s, ia_s,
                           out_dtype=torch.float32 if f32 else torch.bfloat16,
                           split_tokens=split if f32 else None)
    ref = O.grouped_wgrad(u8(go_q), u8(go_s), u8(ia_q), u8(ia_s), ends)
    for g, s in enumerate(sizes):
        if s == 0:
            assert torch.all(dw[g] == 0)
        else:
            assert_close_to_oracle(dw[g], ref[g])


def _cast_cases(n=12, seed=300):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        E = int(rng.integers(1, 20))
        M = int(rng.integers(1, 900))
        out.append((_sizes(rng, E, M), 32 * int(rng.integers(1, 21)),
                    ["rceil", "floor"][int(rng.integers(0, 2))], int(rng.integers(0, 2**31))))
    return out


@pytest.mark.parametrize("sizes,C,mode_name,seed", _cast_cases())
def test_random_dual_cast(gpu, sizes, C, mode_name, seed):
    mode = O.RCEIL if mode_name == "rceil" else O.FLOOR
    M = sum(sizes)
    g = torch.Generator(device=gpu).manual_seed(seed)
    x = (torch.randn(M, C, generator=g, device=gpu) *
         torch.exp2(torch.randint(-20, 20, (M, 1), generator=g, device=gpu).float())).to(torch.bfloat16)
    if M > 2:
        x[M // 2, C // 3] = float("nan")
        x[M // 3, C - 1] = float("-inf")
    ends = workloads.ends_of(sizes)
    q, s, qt, st, pad = mxfp8gg.to_mxfp8_dual(x, torch.from_numpy(ends).to(gpu), mode_name)
    rq, rs = O.quant_dim0(bits(x), mode)
    assert np.array_equal(u8(q), rq) and np.array_equal(u8(s), rs)
    rqt, rst, rpad = O.quant_dim1(bits(x), ends, qt.shape[1], mode)
    assert np.array_equal(u8(qt), rqt) and np.array_equal(u8(st), rst)
    assert np.array_equal(pad.cpu().numpy(), rpad)


def _swiglu_cases(n=10, seed=350):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        E = int(rng.integers(1, 9))
        M = int(rng.integers(1, 700))
        out.append((_sizes(rng, E, M), 128 * int(rng.integers(1, 4)), 32 * int(rng.integers(1, 13)),
                    bool(rng.integers(0, 2)), ["rceil", "floor"][int(rng.integers(0, 2))],
                    int(rng.integers(0, 2**31))))
    return out


@pytest.mark.parametrize("sizes,F,K,scaled,mode,seed", _swiglu_cases())
def test_random_fused_swiglu_forward(gpu, sizes, F, K, scaled, mode, seed):
    E, M = len(sizes), sum(sizes)
    a_q, a_s = _rand_q((max(M, 1), K), gpu, seed)
    w_q, w_s = _rand_q((E, 2 * F, K), gpu, seed + 1)
    a_q, a_s = a_q[:M], a_s[:M]
    if not scaled:
        a_s = w_s = None
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(gpu)
    f8 = torch.float8_e4m3fn
    args = (a_q.view(f8), w_q.view(f8), offs, a_s, w_s, mode)
    # the fused kernel never splits K: its h is the unsplit GEMM's, bit for bit
    h = ops.grouped_mm(*args[:5], split_tail=False)
    rq, rs = ops.swiglu_quant(h, mode)
    q, s = ops.grouped_mm_swiglu_quant(*args)
    qk, sk, hk = ops.grouped_mm_swiglu_quant(*args, return_h=True)
    assert torch.equal(q.view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(s, rs)
    assert torch.equal(qk.view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(sk, rs)
    assert torch.equal(hk.view(torch.int16), h.view(torch.int16))


def _route_cases(n=12, seed=400):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        out.append((int(rng.integers(0, 3000)), int(rng.integers(1, 12)),
                    int(rng.integers(1, 300)), [1, 4, 32, 128][int(rng.integers(0, 4))],
                    8 * int(rng.integers(1, 20)), int(rng.integers(0, 2**31))))
    return out


@pytest.mark.parametrize("T,K,E,pad,H,seed", _route_cases())
def test_random_routing(gpu, T, K, E, pad, H, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(-1, E + 1, (T, K), generator=g, dtype=torch.int32)  # some dropped
    plan = mxfp8gg.route_plan(idx.to(gpu), E, pad)
    perm, src, ends, counts = O.route_plan(idx.numpy(), E, pad, T * K + E * (pad - 1))
    assert np.array_equal(plan.perm.cpu().numpy(), perm)
    assert np.array_equal(plan.src.cpu().numpy(), src)
    assert np.array_equal(plan.offs.cpu().numpy(), ends)
    assert np.array_equal(plan.counts.cpu().numpy(), counts)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(gpu)
    sc = torch.rand(T, K, generator=g).to(gpu)
    assert np.array_equal(bits(mxfp8gg.gather_rows(x, plan, sc)),
                          O.gather_rows(bits(x), src, K, sc.cpu().numpy()))
    y = torch.randn(plan.rows, H, generator=g).to(torch.bfloat16).to(gpu)
    assert np.array_equal(bits(mxfp8gg.combine(y, plan, sc)),
                          O.combine(bits(y), perm, K, sc.cpu().numpy()))
