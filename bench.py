#!/usr/bin/env python3
"""Benchmark of the MXFP8 grouped-GEMM path on one MI355X.

Headline ("C2"): DeepSeek-V3 gate+up forward on one
GPU's expert share — 32 experts, K=7168, N=4096, 65536 tokens routed by
Multinomial(Dirichlet(1)) — MXFP8 e4m3 operands with E8M0 1x32 scales, bf16
output, fp32 accumulation.  A step is one grouped-GEMM launch over the whole
batch with operands already resident in HBM (quantised once before timing).
value = 2 * tokens * N * K / step time, in TFLOPS.

The same run also times, as secondary components: the C3 down-projection
forward, the C4 weight gradient (fp32 dW), the bf16->MXFP8 casts, and the
reference's CPU path (dequantise + per-group fp32 matmul with torch on the
host cores) on a bounded sample of C2.  Last, roofline.traffic (HBM bytes per
C2 launch) is measured by four rocprofv3 counter passes in child processes
(FETCH_SIZE and WRITE_SIZE over `--only fwd` and over a 1 GiB copy, which
calibrates both counters); --no-traffic skips them.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-traffic]
                      [--only fwd|wgrad|copy|ref8|refwgrad|c5|routing|dense|dense_clock|small|
                              traffic|hbm]
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "mxfp8-grouped-gemm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_MXFP8_TFLOPS = 5000.0  # MI355X dense fp8 / MXFP8 MFMA peak (published)
PEAK_HBM_GBPS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_launches(fn, steps, warmup, torch):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps  # ms per launch


# The reference's published forward numbers on MI355X are geometric means over
# these 8 equal-group DeepSeek-V3 shapes (fused_fwd.py:323-333): 1501 TFLOPS
# with E8M0 scales, 1864 without.
REF_GEOMEAN_SCALED = 1501.0
REF_GEOMEAN_UNSCALED = 1864.0


def ref_equal_shapes(torch, mxfp8gg, workloads, dev, steps=10, warmup=3):
    """Scaled and unscaled forward TFLOPS on the reference's 8 equal-group shapes."""
    import math
    rows = []
    gen = torch.Generator(device=dev).manual_seed(0)
    for E, M, N, K in workloads.DSV3_EQUAL_SHAPES:
        x = torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16)
        w = (torch.randn((E, N, K), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        xq, xs = mxfp8gg.to_mxfp8_dim0(x)
        wq, ws = mxfp8gg.to_mxfp8_dim0(w)
        del x, w
        ends = torch.arange(1, E + 1, dtype=torch.int32, device=dev) * (M // E)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        fl = 2 * M * N * K
        ms_s = time_launches(lambda: mxfp8gg.grouped_mm(xq, wq, ends, xs, ws, out=out),
                             steps, warmup, torch)
        ms_u = time_launches(lambda: mxfp8gg.grouped_mm(xq, wq, ends, out=out), steps, warmup, torch)
        rows.append({"E": E, "M": M, "N": N, "K": K, "scaled_tflops": round(fl / ms_s / 1e9, 1),
                     "unscaled_tflops": round(fl / ms_u / 1e9, 1)})
        del xq, xs, wq, ws, out
    gs = math.exp(sum(math.log(r["scaled_tflops"]) for r in rows) / len(rows))
    gu = math.exp(sum(math.log(r["unscaled_tflops"]) for r in rows) / len(rows))
    return {"shapes": rows, "geomean_scaled_tflops": round(gs, 1),
            "geomean_unscaled_tflops": round(gu, 1),
            "reference_geomean_scaled": REF_GEOMEAN_SCALED,
            "reference_geomean_unscaled": REF_GEOMEAN_UNSCALED,
            "vs_reference_scaled": round(gs / REF_GEOMEAN_SCALED, 3),
            "vs_reference_unscaled": round(gu / REF_GEOMEAN_UNSCALED, 3)}


# The reference's wgrad is published as a geometric mean over the 8 DSv3 shapes
# of bench_wgrad_dsv3.py:10-19 (equal groups, no scales, bf16 dW): 1913 TFLOPS
# (wgrad_fused.py:2) and 1839 TFLOPS (memory/2026-06-10.md:100).
REF_WGRAD_SHAPES = [  # (name, E, N, K, M) as in bench_wgrad_dsv3.py:10-19
    ("gate_up", 4, 2048, 7168, 32768), ("down", 4, 7168, 2048, 32768),
    ("gate_up", 4, 2048, 7168, 128000), ("down", 4, 7168, 2048, 128000),
    ("gate_up", 8, 2048, 7168, 32768), ("down", 8, 7168, 2048, 32768),
    ("gate_up", 8, 2048, 7168, 128000), ("down", 8, 7168, 2048, 128000),
]
REF_WGRAD_GEOMEANS = (1913.0, 1839.0)


def ref_wgrad_shapes(torch, mxfp8gg, dev, steps=10, warmup=3):
    """Weight gradient on the reference's own 8 wgrad shapes: operands cast as
    bench_wgrad_dsv3.py:41-52 does (go = dY^T [N, M], ia = X^T [K, M], randn,
    offs = [M/E] * E group sizes) and called through the reference-named
    wgrad_prepare / wgrad_kernel; unscaled (the published configuration) and
    with E8M0 scales (token-axis casts), bf16 dW (what wgrad_kernel returns)
    and fp32 dW."""
    import math
    from mxfp8gg import ops
    rows = []
    gen = torch.Generator(device=dev).manual_seed(3)
    for name, E, N, K, M in REF_WGRAD_SHAPES:
        mg = M // E
        dy = torch.randn((M, N), generator=gen, device=dev).to(torch.bfloat16)
        x = torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16)
        go8 = dy.t().contiguous().to(torch.float8_e4m3fn)
        ia8 = x.t().contiguous().to(torch.float8_e4m3fn)
        sizes = torch.full((E,), mg, dtype=torch.int32, device=dev)
        data = mxfp8gg.wgrad_prepare(go8, ia8, sizes)
        ends = torch.arange(1, E + 1, dtype=torch.int32, device=dev) * mg
        go, gos, pad = mxfp8gg.to_mxfp8_dim1(dy, ends)
        ia, ias, _ = mxfp8gg.to_mxfp8_dim1(x, ends)
        del dy, x
        fl = 2 * M * N * K
        row = {"shape": name, "E": E, "N": N, "K": K, "M": M}
        for dt, tag in ((torch.bfloat16, "bf16"), (torch.float32, "f32")):
            out = torch.empty((E, N, K), dtype=dt, device=dev)
            ms_u = time_launches(
                lambda: ops.grouped_wgrad(data["A"], data["B"], data["offs"], out_dtype=dt,
                                          out=out), steps, warmup, torch)
            ms_s = time_launches(
                lambda: ops.grouped_wgrad(go, ia, pad, gos, ias, out_dtype=dt, out=out),
                steps, warmup, torch)
            row[f"unscaled_{tag}_tflops"] = round(fl / ms_u / 1e9, 1)
            row[f"scaled_{tag}_tflops"] = round(fl / ms_s / 1e9, 1)
            del out
        rows.append(row)
        del go8, ia8, go, gos, ia, ias, data
    res = {"shapes": rows}
    for key in ("unscaled_bf16", "scaled_bf16", "unscaled_f32", "scaled_f32"):
        res[f"geomean_{key}_tflops"] = round(
            math.exp(sum(math.log(r[f"{key}_tflops"]) for r in rows) / len(rows)), 1)
    res["reference_geomeans"] = list(REF_WGRAD_GEOMEANS)
    res["vs_reference_unscaled_bf16"] = [round(res["geomean_unscaled_bf16_tflops"] / r, 3)
                                         for r in REF_WGRAD_GEOMEANS]
    return res


def dense_c2_shape(torch, mxfp8gg, dev, steps=10, warmup=3):
    """C2's GEMM as one dense group (M=65536, N=4096, K=7168): this library's
    kernel with and without E8M0 scales, and the vendor library through
    torch._scaled_mm (hipBLASLt) at the same shape, tensorwise fp8 and MX
    block-scaled, for reference.  Separates the kernel's own ceiling from what
    C2's ragged groups cost (partial m-tiles, a last round of tiles)."""
    M, N, K = 65536, 4096, 7168
    gen = torch.Generator(device=dev).manual_seed(0)
    xq, xs = mxfp8gg.to_mxfp8_dim0(torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16))
    wq, ws = mxfp8gg.to_mxfp8_dim0(
        (torch.randn((1, N, K), generator=gen, device=dev) * 0.006).to(torch.bfloat16))
    ends = torch.tensor([M], dtype=torch.int32, device=dev)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    fl = 2 * M * N * K

    one = torch.ones((), device=dev)
    e8 = torch.float8_e8m0fnu
    sa, sb = xs.contiguous().view(e8), ws[0].contiguous().view(e8)
    cases = {
        "mxgg_scaled_tflops": lambda: mxfp8gg.grouped_mm(xq, wq, ends, xs, ws, out=out),
        "mxgg_unscaled_tflops": lambda: mxfp8gg.grouped_mm(xq, wq, ends, out=out),
        "hipblaslt_fp8_tensorwise_tflops":
            lambda: torch._scaled_mm(xq, wq[0].t(), one, one, out_dtype=torch.bfloat16),
        "hipblaslt_mxfp8_tflops":
            lambda: torch._scaled_mm(xq, wq[0].t(), sa, sb, out_dtype=torch.bfloat16)}
    res = {"M": M, "N": N, "K": K, "note": "best of 3 interleaved rounds"}
    best = {}
    for _ in range(3):   # interleaved, so clock and thermal drift hit every case alike
        for name, fn in cases.items():
            if isinstance(best.get(name), str):
                continue
            try:
                t = round(fl / time_launches(fn, steps, warmup, torch) / 1e9, 1)
                best[name] = max(best.get(name, 0.0), t)
            except Exception as ex:  # the vendor paths are a comparison only
                best[name] = "unavailable: " + str(ex)[:120]
    res.update(best)
    return res


def _sclk_mhz():
    """Current shader clock of card 0 from rocm-smi (MHz), or None."""
    import re
    import subprocess
    try:
        r = subprocess.run(["rocm-smi", "-d", "0", "--showclocks", "--json"],
                           capture_output=True, text=True, timeout=20)
        card = json.loads(r.stdout)["card0"]
        return int(re.search(r"(\d+)", card["sclk clock speed:"]).group(1))
    except Exception:  # the clock is context for the rates, not a result
        return None


def dense_sustained(torch, mxfp8gg, dev, seconds=5.0):
    """The dense C2 shape run back to back for `seconds` per case (this
    library's kernel with and without E8M0 scales, hipBLASLt's tensorwise fp8
    kernel through torch._scaled_mm), with the shader clock sampled by rocm-smi
    while each runs.  Under sustained load the chip is power-limited, so the
    clock (and TFLOPS per GHz) separates cycles from clock."""
    import threading
    M, N, K = 65536, 4096, 7168
    gen = torch.Generator(device=dev).manual_seed(0)
    xq, xs = mxfp8gg.to_mxfp8_dim0(torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16))
    wq, ws = mxfp8gg.to_mxfp8_dim0(
        (torch.randn((1, N, K), generator=gen, device=dev) * 0.006).to(torch.bfloat16))
    ends = torch.tensor([M], dtype=torch.int32, device=dev)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    one = torch.ones((), device=dev)
    fl = 2 * M * N * K
    cases = {
        "mxgg_scaled": lambda: mxfp8gg.grouped_mm(xq, wq, ends, xs, ws, out=out),
        "mxgg_unscaled": lambda: mxfp8gg.grouped_mm(xq, wq, ends, out=out),
        "hipblaslt_fp8_tensorwise":
            lambda: torch._scaled_mm(xq, wq[0].t(), one, one, out_dtype=torch.bfloat16)}
    res = {"M": M, "N": N, "K": K, "seconds_per_case": seconds, "cases": {}}
    for name, fn in cases.items():
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        clocks, done = [], threading.Event()

        def sample():
            if not done.wait(1.5):           # past the clock's settling time
                while not done.is_set():
                    c = _sclk_mhz()
                    if c is not None:
                        clocks.append(c)
                    done.wait(0.3)
        th = threading.Thread(target=sample)
        th.start()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        n, t0 = 0, time.time()
        start.record()
        while time.time() - t0 < seconds:
            for _ in range(50):
                fn()
            n += 50
            torch.cuda.synchronize()
        stop.record()
        torch.cuda.synchronize()
        done.set()
        th.join()
        ms = start.elapsed_time(stop) / n
        tf = fl / ms / 1e9
        clocks.sort()
        mhz = clocks[len(clocks) // 2] if clocks else None
        res["cases"][name] = {"launches": n, "ms": round(ms, 4), "tflops": round(tf, 1),
                              "sclk_mhz_median": mhz, "sclk_samples": len(clocks),
                              "tflops_per_ghz": round(tf / (mhz / 1000), 1) if mhz else None}
    return res


def small_launches(torch, mxfp8gg, dev, steps=10, warmup=3):
    """Calls with fewer output tiles than compute units, split along K over the
    idle units or not: forward (one expert, K=7168; 16 and 128 tiles) and
    weight gradient (fp32 dW; 32, 64 and 128 tiles, 65536 or 32768 tokens
    spread evenly).  Split forwards/wgrads write fp32 partials to a workspace
    and a second kernel adds them in a fixed order."""
    from mxfp8gg import ops
    res = {"forward": [], "wgrad": []}
    gen = torch.Generator(device=dev).manual_seed(2)
    for M, N in ((512, 2048), (2048, 4096)):
        K = 7168
        xq, xs = mxfp8gg.to_mxfp8_dim0(torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16))
        wq, ws = mxfp8gg.to_mxfp8_dim0(
            (torch.randn((1, N, K), generator=gen, device=dev) * 0.006).to(torch.bfloat16))
        ends = torch.tensor([M], dtype=torch.int32, device=dev)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        fl = 2 * M * N * K
        row = {"M": M, "N": N, "K": K, "tiles": (M // 256) * (N // 256)}
        for name, sp in (("unsplit_tflops", False), ("split_tflops", True)):
            row[name] = round(fl / time_launches(
                lambda sp=sp: ops.grouped_mm(xq, wq, ends, xs, ws, out=out, split_tail=sp),
                steps, warmup, torch) / 1e9, 1)
        res["forward"].append(row)
    for E, M, N, K in ((2, 65536, 1024, 1024), (1, 32768, 2048, 2048), (4, 65536, 2048, 1024)):
        dy = torch.randn((M, N), generator=gen, device=dev).to(torch.bfloat16)
        x = torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16)
        offs = torch.arange(1, E + 1, dtype=torch.int32, device=dev) * (M // E)
        go, gos, pad = mxfp8gg.to_mxfp8_dim1(dy, offs)
        ia, ias, _ = mxfp8gg.to_mxfp8_dim1(x, offs)
        del dy, x
        out = torch.empty((E, N, K), dtype=torch.float32, device=dev)
        split = ops.wgrad_split_tokens(go.shape[1], N, K, E, ops._cu_count(dev))
        fl = 2 * M * N * K
        row = {"E": E, "tokens": M, "N": N, "K": K, "tiles": E * (N // 256) * (K // 256),
               "split_tokens": split}
        for name, sp in (("unsplit_tflops", 0), ("split_tflops", split)):
            row[name] = round(fl / time_launches(
                lambda sp=sp: ops.grouped_wgrad(go, ia, pad, gos, ias, out=out, split_tokens=sp),
                steps, warmup, torch) / 1e9, 1)
        res["wgrad"].append(row)
    return res


def layer_step_c5(torch, mxfp8gg, workloads, dev, steps=5, warmup=2):
    """one DSv3 expert-FFN layer step on one GPU --
    131072 routed tokens, Zipf(1.0) over 32 experts, hidden 7168, intermediate
    2048 -- forward (casts, gate+up, SiLU*up, down) and backward (dgrad and
    wgrad of both projections with their casts) through mxfp8gg.moe_ffn.
    TFLOPS counts the six GEMMs: 18 * tokens * 2048 * 7168 FLOP."""
    sizes = workloads.c5_sizes()
    M, H, F, E = int(sizes.sum()), 7168, 2048, 32
    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((M, H), generator=gen, device=dev).to(torch.bfloat16).requires_grad_(True)
    wgu = (torch.randn((E, 2 * F, H), generator=gen, device=dev) * 0.006).to(torch.bfloat16)
    wd = (torch.randn((E, H, F), generator=gen, device=dev) * 0.006).to(torch.bfloat16)
    wgu.requires_grad_(True)
    wd.requires_grad_(True)
    dy = (torch.randn((M, H), generator=gen, device=dev) * 1e-3).to(torch.bfloat16)
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(dev)

    def step():
        for t in (x, wgu, wd):
            t.grad = None
        mxfp8gg.moe_ffn(x, wgu, wd, offs).backward(dy)

    def fwd():
        with torch.no_grad():
            mxfp8gg.moe_ffn(x, wgu, wd, offs)

    def step_unfused():
        for t in (x, wgu, wd):
            t.grad = None
        mxfp8gg.moe_ffn_unfused(x, wgu, wd, offs).backward(dy)

    ms = time_launches(step, steps, warmup, torch)
    ms_f = time_launches(fwd, steps, warmup, torch)
    ms_u = time_launches(step_unfused, steps, warmup, torch)
    flops = 18 * M * F * H
    out = {"ms": round(ms, 3), "tflops": round(flops / ms / 1e9, 1),
           "frac_of_peak": round(flops / ms / 1e9 / PEAK_MXFP8_TFLOPS, 4),
           "fwd_ms": round(ms_f, 3), "fwd_tflops": round(flops / 3 / ms_f / 1e9, 1),
           "unfused_activation_ms": round(ms_u, 3),
           "tokens": M, "group_sizes_min_max": [int(sizes.min()), int(sizes.max())]}
    for t in (x, wgu, wd):
        t.grad = None
    del wgu, wd
    # the two SwiGLU kernels alone at this shape (HBM-bound; algorithmic bytes:
    # forward reads h and writes a's cast, backward reads h and dA and writes
    # three casts)
    h = torch.randn((M, 2 * F), generator=gen, device=dev).to(torch.bfloat16)
    da = (torch.randn((M, F), generator=gen, device=dev) * 0.05).to(torch.bfloat16)
    cap = mxfp8gg.padded_token_capacity(M, E)
    ms_sf = time_launches(lambda: mxfp8gg.swiglu_quant(h), 10, 3, torch)
    ms_sb = time_launches(lambda: mxfp8gg.swiglu_backward_quant(h, da, offs), 10, 3, torch)
    cast = 1 + 1 / 32
    b_fwd = M * 2 * F * 2 + M * F * cast
    b_bwd = M * 2 * F * 2 + M * F * 2 + M * 2 * F * cast + 3 * F * cap * cast
    out["swiglu_fwd"] = {"ms": round(ms_sf, 4), "GBps": round(b_fwd / ms_sf / 1e6, 1)}
    out["swiglu_bwd"] = {"ms": round(ms_sb, 4), "GBps": round(b_bwd / ms_sb / 1e6, 1)}
    del x, dy, h, da
    return out


def hbm_ceiling(torch, mxfp8gg, workloads, dev, steps=10, warmup=3):
    """What plain device kernels reach on this box's HBM, next to the casts on
    the same data: torch's fill_ (write), sum and amax (read), copy_ (read +
    write) of 2 GiB, and torch's own bf16 -> fp8 conversion (2 bytes read, 1
    written per element: the casts' traffic mix without the scales) of C2's X
    (65536 x 7168), against this library's row-wise, token-axis and dual casts
    of that X, and its two SwiGLU kernels at C5's shape.  GB/s counts
    algorithmic bytes."""
    nb = 2 << 30
    a = torch.empty(nb, dtype=torch.uint8, device=dev)
    b = torch.empty(nb, dtype=torch.uint8, device=dev)
    a.fill_(1)
    res = {}
    ms = time_launches(lambda: b.fill_(3), steps, warmup, torch)
    res["write_fill"] = {"GBps": round(nb / ms / 1e6, 1)}
    af = a.view(torch.float32)
    ms = time_launches(lambda: af.sum(), steps, warmup, torch)
    res["read_sum"] = {"GBps": round(nb / ms / 1e6, 1)}
    ms = time_launches(lambda: af.amax(), steps, warmup, torch)
    res["read_amax"] = {"GBps": round(nb / ms / 1e6, 1)}
    ms = time_launches(lambda: b.copy_(a), steps, warmup, torch)
    res["copy"] = {"GBps": round(2 * nb / ms / 1e6, 1)}
    del a, b, af
    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((65536, 7168), generator=gen, device=dev).to(torch.bfloat16)
    n = x.numel()
    ms = time_launches(lambda: x.to(torch.float8_e4m3fn), steps, warmup, torch)
    res["torch_bf16_to_fp8"] = {"GBps": round(3 * n / ms / 1e6, 1), "bytes_per_elt": 3}
    ms = time_launches(lambda: mxfp8gg.to_mxfp8_dim0(x), steps, warmup, torch)
    res["mxgg_quant_dim0"] = {"GBps": round((3 + 1 / 32) * n / ms / 1e6, 1),
                              "bytes_per_elt": 3.03125}
    offs = torch.tensor([65536], dtype=torch.int32, device=dev)
    ms = time_launches(lambda: mxfp8gg.to_mxfp8_dual(x, offs), steps, warmup, torch)
    res["mxgg_quant_dual"] = {"GBps": round((2 + 2 * (1 + 1 / 32)) * n / ms / 1e6, 1),
                              "bytes_per_elt": 4.0625}
    ms = time_launches(lambda: mxfp8gg.to_mxfp8_dim1(x, offs), steps, warmup, torch)
    res["mxgg_quant_dim1"] = {"GBps": round((3 + 1 / 32) * n / ms / 1e6, 1),
                              "bytes_per_elt": 3.03125}
    del x
    # the SwiGLU kernels at C5's shape (131072 tokens, intermediate 2048,
    # Zipf(1.0) groups): forward reads h [M, 2F] and writes a's cast; backward
    # reads h and dA and writes the row-wise cast of dh and the token-axis
    # casts of dh and a
    sizes = workloads.c5_sizes()
    M, F = int(sizes.sum()), 2048
    e5 = torch.from_numpy(workloads.ends_of(sizes)).to(dev)
    cap = mxfp8gg.padded_token_capacity(M, len(sizes))
    h = torch.randn((M, 2 * F), generator=gen, device=dev).to(torch.bfloat16)
    da = (torch.randn((M, F), generator=gen, device=dev) * 0.05).to(torch.bfloat16)
    cast = 1 + 1 / 32
    ms = time_launches(lambda: mxfp8gg.swiglu_quant(h), steps, warmup, torch)
    res["mxgg_swiglu_fwd_c5"] = {"GBps": round((M * 2 * F * 2 + M * F * cast) / ms / 1e6, 1)}
    ms = time_launches(lambda: mxfp8gg.swiglu_backward_quant(h, da, e5), steps, warmup, torch)
    b_bwd = M * 2 * F * 2 + M * F * 2 + M * 2 * F * cast + 3 * F * cap * cast
    res["mxgg_swiglu_bwd_c5"] = {"GBps": round(b_bwd / ms / 1e6, 1)}
    del h, da
    return res


def gate_up_swiglu_c5(torch, mxfp8gg, workloads, dev, steps=10, warmup=3):
    """C5's gate+up projection (131072 tokens, Zipf(1.0) over 32 experts,
    hidden 7168, intermediate 2048) four ways: the grouped GEMM alone (bf16
    h [M, 4096]), GEMM + the standalone SwiGLU cast (the unfused sequence),
    the fused kernel that writes only the MXFP8 cast of SiLU(gate) * up (the
    forward-only pass), and the fused kernel that also writes bf16 h (the
    training forward)."""
    from mxfp8gg import ops
    sizes = workloads.c5_sizes()
    M, H, F, E = int(sizes.sum()), 7168, 2048, 32
    gen = torch.Generator(device=dev).manual_seed(0)
    xq, xs = mxfp8gg.to_mxfp8_dim0(torch.randn((M, H), generator=gen, device=dev).to(torch.bfloat16))
    wq, ws = mxfp8gg.to_mxfp8_dim0(
        (torch.randn((E, 2 * F, H), generator=gen, device=dev) * 0.006).to(torch.bfloat16))
    offs = torch.from_numpy(workloads.ends_of(sizes)).to(dev)
    h = torch.empty((M, 2 * F), dtype=torch.bfloat16, device=dev)
    fl = 2 * M * 2 * F * H
    ms_g = time_launches(lambda: ops.grouped_mm(xq, wq, offs, xs, ws, out=h), steps, warmup, torch)
    ms_u = time_launches(lambda: ops.swiglu_quant(ops.grouped_mm(xq, wq, offs, xs, ws, out=h)),
                         steps, warmup, torch)
    ms_f = time_launches(lambda: ops.grouped_mm_swiglu_quant(xq, wq, offs, xs, ws), steps, warmup,
                         torch)
    del h
    ms_k = time_launches(lambda: ops.grouped_mm_swiglu_quant(xq, wq, offs, xs, ws, return_h=True),
                         steps, warmup, torch)
    return {"tokens": M, "gemm_bf16_h_ms": round(ms_g, 4),
            "gemm_bf16_h_tflops": round(fl / ms_g / 1e9, 1),
            "gemm_then_swiglu_cast_ms": round(ms_u, 4),
            "fused_ms": round(ms_f, 4), "fused_tflops": round(fl / ms_f / 1e9, 1),
            "fused_keep_h_ms": round(ms_k, 4), "fused_keep_h_tflops": round(fl / ms_k / 1e9, 1)}


def routing_c5(torch, mxfp8gg, workloads, dev, steps=5, warmup=2):
    """C5 as a routed MoE layer: 16384 tokens x top-8 over 32 experts (Zipf(1.0)
    preference), hidden 7168, intermediate 2048.  Times the device dispatch
    plan, the dual MXFP8 cast gathered from token order (against the gather
    and the plain dual cast of the routed rows it replaces), the score-weighted
    combine and its score gradient, and the whole routed layer step (plan,
    casts, six GEMMs, SwiGLU, combine; forward + backward) through
    mxfp8gg.moe_routed_ffn, and its forward-only pass (no autograd, weight
    casts cached: the inference step).  Bytes are algorithmic: bf16 rows read and
    written, 1 + 1/32 bytes per element of each MXFP8 cast."""
    idx_np, sc_np = workloads.c5_routing()
    T, K = idx_np.shape
    H, F, E = 7168, 2048, 32
    idx = torch.from_numpy(idx_np).to(dev)
    sc = torch.from_numpy(sc_np).to(dev)
    gen = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn((T, H), generator=gen, device=dev).to(torch.bfloat16)
    plan = mxfp8gg.route_plan(idx, E)
    rows, slots, cast = plan.rows, T * K, 1 + 1 / 32
    ms_plan = time_launches(lambda: mxfp8gg.route_plan(idx, E), 20, 3, torch)
    ms_gd = time_launches(lambda: mxfp8gg.gather_to_mxfp8_dual(x, plan), 10, 3, torch)
    ms_g = time_launches(lambda: mxfp8gg.gather_rows(x, plan), 10, 3, torch)
    xr = mxfp8gg.gather_rows(x, plan)
    ms_d = time_launches(lambda: mxfp8gg.to_mxfp8_dual(xr, plan.offs), 10, 3, torch)
    del xr
    ms_g0 = time_launches(lambda: mxfp8gg.gather_to_mxfp8_dim0(x, plan), 10, 3, torch)
    b_dual = rows * H * (2 + 2 * cast)
    b_dim0 = rows * H * (2 + cast)
    y = torch.randn((rows, H), generator=gen, device=dev).to(torch.bfloat16)
    d = torch.randn((T, H), generator=gen, device=dev).to(torch.bfloat16)
    ms_c = time_launches(lambda: mxfp8gg.combine(y, plan, sc), 10, 3, torch)
    ms_sg = time_launches(lambda: mxfp8gg.combine_score_grad(d, y, plan), 10, 3, torch)
    del y
    b_comb = slots * H * 2 + T * H * 2
    out = {"tokens": T, "topk": K, "routed_rows": slots, "layout_rows": rows,
           "route_plan_us": round(ms_plan * 1e3, 1),
           "gather_dual_cast": {"ms": round(ms_gd, 4), "GBps": round(b_dual / ms_gd / 1e6, 1)},
           "gather_then_dual_cast_ms": round(ms_g + ms_d, 4),
           "gather_dim0_cast": {"ms": round(ms_g0, 4), "GBps": round(b_dim0 / ms_g0 / 1e6, 1)},
           "combine": {"ms": round(ms_c, 4), "GBps": round(b_comb / ms_c / 1e6, 1)},
           "combine_score_grad": {"ms": round(ms_sg, 4), "GBps": round(b_comb / ms_sg / 1e6, 1)}}
    wgu = (torch.randn((E, 2 * F, H), generator=gen, device=dev) * 0.006).to(torch.bfloat16)
    wd = (torch.randn((E, H, F), generator=gen, device=dev) * 0.006).to(torch.bfloat16)
    leaves = [t.requires_grad_(True) for t in (x, sc, wgu, wd)]

    def step():
        for t in leaves:
            t.grad = None
        mxfp8gg.moe_routed_ffn(x, idx, sc, wgu, wd).backward(d)

    ms = time_launches(step, steps, warmup, torch)
    flops = 18 * slots * F * H
    out["layer_step"] = {"ms": round(ms, 3), "tflops": round(flops / ms / 1e9, 1),
                         "frac_of_peak": round(flops / ms / 1e9 / PEAK_MXFP8_TFLOPS, 4)}
    cache = mxfp8gg.WeightCastCache()

    def fwd():
        with torch.no_grad():
            mxfp8gg.moe_routed_ffn(x, idx, sc, wgu, wd, weight_cache=cache)

    ms_f = time_launches(fwd, steps, warmup, torch)
    flops_f = 6 * slots * F * H
    out["forward_only_cached_weights"] = {
        "ms": round(ms_f, 3), "tflops": round(flops_f / ms_f / 1e9, 1),
        "frac_of_peak": round(flops_f / ms_f / 1e9 / PEAK_MXFP8_TFLOPS, 4)}
    del cache
    for t in leaves:
        t.grad = None
    return out


GEMM_SOURCE = ROOT / "mxfp8-grouped-gemm_amd" / "csrc" / "gemm.hip"
# every file the GEMM translation unit includes from the tree, so an edit to a
# shared device helper also marks a stored traffic figure stale
GEMM_HEADERS = [ROOT / "mxfp8-grouped-gemm_amd" / "csrc" / "mx_device.h",
                ROOT / "mxfp8-grouped-gemm_amd" / "csrc" / "mxgg_internal.h",
                ROOT / "include" / "mxgg.h"]
TRAFFIC_FILE = ROOT / "profiles" / "traffic_grouped_fwd_c2.json"
HEADLINE_KERNEL = "k_grouped_fwd"   # the C2 launch: k_grouped_fwd<true, 0> (scaled, bf16 out)


def _source_hash():
    import hashlib
    h = hashlib.sha256()
    for f in [GEMM_SOURCE] + GEMM_HEADERS:
        h.update(f.name.encode() + b"\0" + f.read_bytes())
    return h.hexdigest()


def _pmc_pass(only, counter, out_dir):
    """One rocprofv3 counter pass over `bench.py --only <only>` in a child
    process; returns {kernel name: (mean counter value per dispatch, dispatches)}."""
    import csv
    import shutil
    import subprocess
    shutil.rmtree(out_dir, ignore_errors=True)
    cmd = ["timeout", "-s", "KILL", "75", "rocprofv3", "--pmc", counter, "--output-format", "csv",
           "-d", str(out_dir), "-o", "p", "--", sys.executable, str(ROOT / "bench.py"),
           "--only", only, "--steps", "3", "--warmup", "1", "--no-cpu"]
    log("traffic pass: " + " ".join(cmd))
    subprocess.run(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"), check=False,
                   stdout=subprocess.DEVNULL)
    files = sorted(Path(out_dir).rglob("*counter_collection.csv"))
    if not files:
        raise RuntimeError(f"rocprofv3 wrote no counter file under {out_dir}")
    tot, ids = {}, {}
    for r in csv.DictReader(open(files[0])):
        k = r["Kernel_Name"]
        tot[k] = tot.get(k, 0.0) + float(r["Counter_Value"])
        ids.setdefault(k, set()).add(r["Dispatch_Id"])
    return {k: (tot[k] / len(ids[k]), len(ids[k])) for k in tot}


def measure_traffic():
    """HBM bytes per launch of the headline kernel from rocprofv3 FETCH_SIZE and
    WRITE_SIZE passes (KiB per dispatch), each scaled by what the same counter
    reads for a 1 GiB device copy, written to profiles/ with the hash of the
    kernel source it was measured on.  Raises if a pass yields no counters."""
    import tempfile
    res = {}
    with tempfile.TemporaryDirectory(prefix="mxgg_traffic_", dir="/tmp") as tmp:
        for only in ("fwd", "copy"):
            for counter in ("FETCH_SIZE", "WRITE_SIZE"):
                res[(only, counter)] = _pmc_pass(only, counter, Path(tmp) / f"{only}_{counter}")
                if not res[(only, counter)]:
                    raise RuntimeError(f"rocprofv3 {counter} pass over --only {only} gave no counters")
    names = {c: next(k for k in res[("fwd", c)] if HEADLINE_KERNEL in k)
             for c in ("FETCH_SIZE", "WRITE_SIZE")}
    fwd = {c: res[("fwd", c)][names[c]] for c in ("FETCH_SIZE", "WRITE_SIZE")}
    cp = {c: max(res[("copy", c)].values()) for c in ("FETCH_SIZE", "WRITE_SIZE")}
    nbytes = 1 << 30
    ff = nbytes / (cp["FETCH_SIZE"][0] * 1024)
    wf = nbytes / (cp["WRITE_SIZE"][0] * 1024)
    rd = fwd["FETCH_SIZE"][0] * 1024 * ff
    wr = fwd["WRITE_SIZE"][0] * 1024 * wf
    out = {
        "kernel": names["FETCH_SIZE"] + " on C2 (65536 tokens, 32 experts, K=7168, N=4096)",
        "kernel_source": [str(f.relative_to(ROOT)) for f in [GEMM_SOURCE] + GEMM_HEADERS],
        "kernel_source_sha256": _source_hash(),
        "hbm_bytes_per_launch": int(rd + wr),
        "hbm_read_bytes": int(rd), "hbm_write_bytes": int(wr),
        "fetch_size_kib_per_dispatch": fwd["FETCH_SIZE"][0],
        "write_size_kib_per_dispatch": fwd["WRITE_SIZE"][0],
        "calibration": {"copy_bytes_read": nbytes, "copy_bytes_written": nbytes,
                        "copy_fetch_size_kib": cp["FETCH_SIZE"][0],
                        "copy_write_size_kib": cp["WRITE_SIZE"][0],
                        "fetch_factor": round(ff, 4), "write_factor": round(wf, 4)},
        "algorithmic_bytes_per_launch": 1990197248,
        "command": "python3 bench.py --only traffic",
    }
    TRAFFIC_FILE.write_text(json.dumps(out, indent=1) + "\n")
    return out


def stored_traffic():
    """The traffic figure of profiles/ when it was measured on the current
    kernel source, else None (a changed kernel needs `bench.py --only traffic`)."""
    if not TRAFFIC_FILE.exists():
        return None, "no traffic measurement under profiles/"
    t = json.loads(TRAFFIC_FILE.read_text())
    if t.get("kernel_source_sha256") != _source_hash():
        return None, "stale: kernel source changed since the measurement (bench.py --only traffic)"
    return t.get("hbm_bytes_per_launch"), "rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated"


def stored_traffic_kernel():
    """Kernel name the stored traffic figure was counted on (None if absent)."""
    if not TRAFFIC_FILE.exists():
        return None
    return json.loads(TRAFFIC_FILE.read_text()).get("kernel")


def cpu_baseline(xq, xs, wq, ws, ends_np, n, k, gpu_out=None, budget_s=12.0):
    """The reference's CPU path on a bounded sample of the workload: whole
    experts of C2, in order, until `budget_s` of CPU work has run.  With the
    GPU's output of the same launch, also the largest error of its sampled
    rows against that CPU result, max|gpu - cpu| / max|cpu| per expert (the
    normwise measure of the parity tests, bound 1e-2)."""
    import torch
    from oracle import oracle as O

    done_tokens = 0
    t_total = 0.0
    experts = 0
    worst = 0.0
    b = 0
    for g, e in enumerate(ends_np.tolist()):
        if e > b:
            a_q = xq[b:e].cpu().view(torch.uint8)
            a_s = xs[b:e].cpu()
            w_q = wq[g:g + 1].cpu().view(torch.uint8)
            w_s = ws[g:g + 1].cpu()
            t0 = time.perf_counter()
            ref = O.cpu_baseline_fwd(a_q, a_s, w_q, w_s, torch.tensor([e - b], dtype=torch.int32))
            t_total += time.perf_counter() - t0
            if gpu_out is not None:
                got = gpu_out[b:e].float().cpu()
                worst = max(worst, float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30)))
            done_tokens += e - b
            experts += 1
        b = e
        if t_total >= budget_s:
            break
    tflops = 2.0 * done_tokens * n * k / t_total / 1e12
    res = {
        "value": round(tflops, 4),
        "unit": "TFLOPS",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"C2 experts 0..{experts - 1} ({done_tokens} tokens x N={n} x K={k}): "
                  f"dequantise e4m3*2^(b-127) to fp32, per-group fp32 matmul, {t_total:.1f} s",
    }
    if gpu_out is not None:
        res["gpu_max_rel_err"] = float(f"{worst:.3e}")
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 counter passes behind roofline.traffic")
    ap.add_argument("--only", choices=["all", "fwd", "wgrad", "copy", "ref8", "refwgrad", "c5",
                                       "routing", "dense", "dense_clock", "small", "traffic",
                                       "hbm"],
                    default="all",
                    help="fwd / wgrad: time only that GEMM (for profiler runs); copy: a plain "
                         "1 GiB device-to-device copy, the reference for HBM byte counters; "
                         "ref8: the reference's 8 equal-group shapes only; refwgrad: its 8 "
                         "wgrad shapes only; c5: the full "
                         "expert-FFN layer step only; routing: C5 as a routed top-8 layer; "
                         "dense: C2's shape as one dense GEMM, with hipBLASLt beside it; "
                         "dense_clock: the same back to back for 5 s per case with the "
                         "shader clock sampled; "
                         "small: launches with fewer tiles than compute units, split or not; "
                         "hbm: plain-kernel HBM rates beside the casts; "
                         "traffic: rocprofv3 FETCH_SIZE / WRITE_SIZE passes of fwd and copy "
                         "(child processes) -> profiles/traffic_grouped_fwd_c2.json")
    args = ap.parse_args()
    if args.only == "traffic":   # no GPU use in this process: rocprofv3 runs children
        print(json.dumps(measure_traffic()), flush=True)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the MXFP8 grouped GEMM shards by expert and "
              "this build runs a single GPU's expert share; --gpus must be 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import mxfp8gg
    from mxfp8gg import workloads

    dev = torch.device("cuda:0")
    mxfp8gg.load_library()

    if args.only == "c5":
        print(json.dumps(layer_step_c5(torch, mxfp8gg, workloads, dev)), flush=True)
        print(json.dumps(gate_up_swiglu_c5(torch, mxfp8gg, workloads, dev)), flush=True)
        return
    if args.only == "routing":
        print(json.dumps(routing_c5(torch, mxfp8gg, workloads, dev)), flush=True)
        return
    if args.only == "small":
        print(json.dumps(small_launches(torch, mxfp8gg, dev)), flush=True)
        return
    if args.only == "dense":
        print(json.dumps(dense_c2_shape(torch, mxfp8gg, dev)), flush=True)
        return
    if args.only == "dense_clock":
        print(json.dumps(dense_sustained(torch, mxfp8gg, dev)), flush=True)
        return
    if args.only == "ref8":
        print(json.dumps(ref_equal_shapes(torch, mxfp8gg, workloads, dev)), flush=True)
        return
    if args.only == "hbm":
        print(json.dumps(hbm_ceiling(torch, mxfp8gg, workloads, dev)), flush=True)
        return
    if args.only == "refwgrad":
        print(json.dumps(ref_wgrad_shapes(torch, mxfp8gg, dev)), flush=True)
        return
    if args.only == "copy":
        nbytes = 1 << 30
        src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        ms = time_launches(lambda: dst.copy_(src), args.steps, args.warmup, torch)
        print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes,
                          "ms": round(ms, 4), "GBps": round(2 * nbytes / ms / 1e6, 1)}),
              flush=True)
        return
    if args.only == "wgrad":
        dy, x4, s4 = workloads.c4(dev)
        e4 = torch.from_numpy(workloads.ends_of(s4)).to(dev)
        go, gos, pad = mxfp8gg.to_mxfp8_dim1(dy, e4)
        ia, ias, _ = mxfp8gg.to_mxfp8_dim1(x4, e4)
        n4, k4 = dy.shape[1], x4.shape[1]
        del dy, x4
        dw = torch.empty((32, n4, k4), dtype=torch.float32, device=dev)
        ms4 = time_launches(
            lambda: mxfp8gg.grouped_wgrad(go, ia, pad, gos, ias, out_dtype=torch.float32, out=dw),
            args.steps, args.warmup, torch)
        f4 = workloads.gemm_flops(int(s4.sum()), n4, k4)
        print(json.dumps({"wgrad_c4_ms": round(ms4, 4), "tflops": round(f4 / ms4 / 1e9, 1)}),
              flush=True)
        return

    # ---- headline: C2 forward ---------------------------------------------
    log("C2: generating and quantising operands")
    x, w, sizes = workloads.c2(dev)
    ends_np = workloads.ends_of(sizes)
    ends = torch.from_numpy(ends_np).to(dev)
    xq, xs = mxfp8gg.to_mxfp8_dim0(x)
    wq, ws = mxfp8gg.to_mxfp8_dim0(w)
    M, K = x.shape
    E, N, _ = w.shape
    flops = workloads.gemm_flops(M, N, K)

    quant_c2 = None
    if args.only == "all":
        # bf16 -> MXFP8 dim0 on X: algorithmic bytes = 2 (in) + 1 (payload) + 1/32 (scale) per element
        ms_q = time_launches(lambda: mxfp8gg.to_mxfp8_dim0(x), 20, 3, torch)
        qbytes = x.numel() * (2 + 1 + 1 / 32)
        quant_c2 = {"ms": round(ms_q, 4), "GBps": round(qbytes / ms_q / 1e6, 1),
                    "frac_of_8TBps": round(qbytes / ms_q / 1e6 / PEAK_HBM_GBPS, 4)}
    del x, w

    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def step():
        mxfp8gg.grouped_mm(xq, wq, ends, xs, ws, out=out)

    log(f"C2: timing {args.steps} steps after {args.warmup} warm-up")
    ms = time_launches(step, args.steps, args.warmup, torch)
    tflops = flops / (ms * 1e-3) / 1e12

    components = {}
    if args.only == "all":
        components["quant_dim0_c2_x"] = quant_c2
        # ---- C3 forward (down projection) --------------------------------
        log("C3: down-projection forward")
        h, w3, s3 = workloads.c3(dev)
        e3 = torch.from_numpy(workloads.ends_of(s3)).to(dev)
        hq, hs = mxfp8gg.to_mxfp8_dim0(h)
        w3q, w3s = mxfp8gg.to_mxfp8_dim0(w3)
        del h, w3
        o3 = torch.empty((hq.shape[0], w3q.shape[1]), dtype=torch.bfloat16, device=dev)
        ms3 = time_launches(lambda: mxfp8gg.grouped_mm(hq, w3q, e3, hs, w3s, out=o3), 20, 5,
                            torch)
        f3 = workloads.gemm_flops(hq.shape[0], w3q.shape[1], hq.shape[1])
        components["fwd_c3"] = {"ms": round(ms3, 4), "tflops": round(f3 / ms3 / 1e9, 1),
                                "frac_of_peak": round(f3 / ms3 / 1e9 / PEAK_MXFP8_TFLOPS, 4)}
        del hq, hs, w3q, w3s, o3
        # ---- C4 wgrad -------------------------------------------------------
        log("C4: weight gradient")
        dy, x4, s4 = workloads.c4(dev)
        e4 = torch.from_numpy(workloads.ends_of(s4)).to(dev)
        ms_d1 = time_launches(lambda: mxfp8gg.to_mxfp8_dim1(dy, e4), 10, 2, torch)
        go, gos, pad = mxfp8gg.to_mxfp8_dim1(dy, e4)
        ia, ias, _ = mxfp8gg.to_mxfp8_dim1(x4, e4)
        d1bytes = dy.numel() * (2 + 1 + 1 / 32)
        components["quant_dim1_c4_dy"] = {"ms": round(ms_d1, 4),
                                          "GBps": round(d1bytes / ms_d1 / 1e6, 1)}
        n4, k4 = dy.shape[1], x4.shape[1]
        del dy, x4
        dw = torch.empty((32, n4, k4), dtype=torch.float32, device=dev)
        ms4 = time_launches(
            lambda: mxfp8gg.grouped_wgrad(go, ia, pad, gos, ias, out_dtype=torch.float32, out=dw),
            10, 3, torch)
        f4 = workloads.gemm_flops(int(s4.sum()), n4, k4)
        components["wgrad_c4"] = {"ms": round(ms4, 4), "tflops": round(f4 / ms4 / 1e9, 1),
                                  "frac_of_peak": round(f4 / ms4 / 1e9 / PEAK_MXFP8_TFLOPS, 4),
                                  "out": "fp32 [32, 4096, 7168]"}
        del go, gos, ia, ias, dw
        log("reference's 8 equal-group shapes")
        components["ref_equal_shapes"] = ref_equal_shapes(torch, mxfp8gg, workloads, dev)
        log("reference's 8 wgrad shapes")
        components["ref_wgrad_shapes"] = ref_wgrad_shapes(torch, mxfp8gg, dev)
        log("C2's shape as one dense GEMM (kernel ceiling, vendor library beside it)")
        components["dense_c2_shape"] = dense_c2_shape(torch, mxfp8gg, dev)
        log("small launches split along K")
        components["small_launches"] = small_launches(torch, mxfp8gg, dev)
        log("C5: expert-FFN layer step (forward + backward)")
        components["layer_step_c5"] = layer_step_c5(torch, mxfp8gg, workloads, dev)
        log("HBM ceiling of plain kernels beside the casts")
        components["hbm_ceiling"] = hbm_ceiling(torch, mxfp8gg, workloads, dev)
        log("C5 gate+up with SwiGLU: unfused vs fused")
        components["gate_up_swiglu_c5"] = gate_up_swiglu_c5(torch, mxfp8gg, workloads, dev)
        log("C5 as a routed top-8 layer (dispatch, combine)")
        components["routing_c5"] = routing_c5(torch, mxfp8gg, workloads, dev)

    traffic, traffic_note = None, "not measured (--no-traffic or a partial run)"
    traffic_kernel = None
    if args.only == "all" and not args.no_traffic:
        # measured in this run: four rocprofv3 counter passes in child processes,
        # after every timed region above
        log("roofline traffic: rocprofv3 FETCH_SIZE / WRITE_SIZE passes of C2 and a copy")
        try:
            measured = measure_traffic()
            traffic, traffic_kernel = measured["hbm_bytes_per_launch"], measured["kernel"]
            traffic_note = ("measured in this run: rocprofv3 FETCH_SIZE + WRITE_SIZE of the "
                            "C2 launch, each scaled by the same counter over a 1 GiB copy")
        except Exception as exc:  # profiler missing or refused: fall back, say so
            log(f"traffic passes failed: {exc}")
            traffic, traffic_note = stored_traffic()
            traffic_kernel = stored_traffic_kernel() if traffic is not None else None
    elif args.only != "all":
        traffic, traffic_note = stored_traffic()
        traffic_kernel = stored_traffic_kernel() if traffic is not None else None

    cpu = None
    if not args.no_cpu and args.only == "all":
        log("CPU baseline (reference CPU path on a bounded sample)")
        cpu = cpu_baseline(xq, xs, wq, ws, ends_np, N, K, gpu_out=out)

    line = {
        "metric": "MXFP8 grouped-GEMM TFLOPS fwd & wgrad, DSv3 32-expert shape; % of MFMA peak",
        "value": round(tflops, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp8_e4m3 (E8M0 1x32 scales, fp32 accumulate, bf16 out)",
        "data": "synthetic",
        "config": {
            "workload": "C2: DSv3 gate+up grouped forward, 32 local experts, K=7168, N=4096, "
                        "65536 tokens, Dirichlet(1) routing, seed 0",
            "experts": E, "tokens": M, "N": N, "K": K,
            "group_sizes_min_max": [int(sizes.min()), int(sizes.max())],
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops, 2),
            "peak": PEAK_MXFP8_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / PEAK_MXFP8_TFLOPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_note,
            "kernel": traffic_kernel or "k_grouped_fwd<true, 0> (one launch per step)",
        },
        "cpu_baseline": cpu,
        "components": components,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
