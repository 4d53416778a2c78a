"""Synthetic workloads of the benchmark configurations (seeded, reproducible).

C1  tiny forward: E=4, K=256, N=512, group sizes [64, 128, 32, 96]
C2  DSv3 gate+up forward: E=32, K=7168, N=4096, 65536 tokens, Dirichlet(1) routing
C3  DSv3 down forward: E=32, K=2048, N=7168, same routing, activations with 1% x20 outliers
C4  DSv3 wgrad: E=32, dY [M, 4096], X [M, 7168], 65536 tokens, Zipf(1.2) routing with
    the two smallest experts emptied, fp32 dW
C5  full MoE layer step: 131072 tokens, Zipf(1.0) routing, hidden 7168, intermediate 2048

The reference's own sweep shapes (8 equal-group DSv3 shapes, fused_fwd.py:323-333)
are in DSV3_EQUAL_SHAPES.
"""
from __future__ import annotations

import numpy as np
import torch

DSV3_EQUAL_SHAPES = [  # (E, M, N, K), equal groups, as swept by the reference
    (4, 32768, 2048, 7168),
    (4, 32768, 7168, 2048),
    (4, 128000, 2048, 7168),
    (4, 128000, 7168, 2048),
    (8, 32768, 2048, 7168),
    (8, 32768, 7168, 2048),
    (8, 128000, 2048, 7168),
    (8, 128000, 7168, 2048),
]


def dirichlet_sizes(tokens: int, experts: int, seed: int = 0, alpha: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    p = rng.dirichlet(np.full(experts, alpha))
    return rng.multinomial(tokens, p).astype(np.int64)


def zipf_sizes(tokens: int, experts: int, s: float, seed: int = 0, empty: int = 0) -> np.ndarray:
    """Zipf(s) routing probabilities p_i ~ 1/i^s; the `empty` least likely
    experts get no tokens; sizes ~ Multinomial(tokens, p)."""
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, experts + 1, dtype=np.float64) ** s
    if empty:
        p[experts - empty:] = 0.0
    p /= p.sum()
    return rng.multinomial(tokens, p).astype(np.int64)


def ends_of(sizes) -> np.ndarray:
    return np.cumsum(np.asarray(sizes, dtype=np.int64)).astype(np.int32)


def _randn(shape, gen, device, scale=1.0):
    return (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * scale).to(
        torch.bfloat16)


def c1(device="cpu"):
    """Tiny forward config: seed 0, X ~ N(0,1) [320, 256], W ~ N(0, 0.02) [4, 512, 256]."""
    gen = torch.Generator(device="cpu").manual_seed(0)
    x = torch.randn(320, 256, generator=gen, dtype=torch.float32).to(torch.bfloat16)
    w = (torch.randn(4, 512, 256, generator=gen, dtype=torch.float32) * 0.02).to(torch.bfloat16)
    sizes = np.array([64, 128, 32, 96])
    return x.to(device), w.to(device), sizes


def c2(device="cuda", seed=0):
    gen = torch.Generator(device=device).manual_seed(seed)
    sizes = dirichlet_sizes(65536, 32, seed)
    x = _randn((65536, 7168), gen, device)
    w = _randn((32, 4096, 7168), gen, device, 0.006)
    return x, w, sizes


def c3(device="cuda", seed=0):
    gen = torch.Generator(device=device).manual_seed(seed + 1)
    sizes = dirichlet_sizes(65536, 32, seed)
    h = torch.randn((65536, 2048), generator=gen, device=device, dtype=torch.float32) * 0.5
    mask = torch.rand((65536, 2048), generator=gen, device=device) < 0.01
    h = torch.where(mask, h * 20.0, h).to(torch.bfloat16)
    w = _randn((32, 7168, 2048), gen, device, 0.006)
    return h, w, sizes


def c4(device="cuda", seed=0):
    gen = torch.Generator(device=device).manual_seed(seed + 2)
    sizes = zipf_sizes(65536, 32, 1.2, seed, empty=2)
    dy = _randn((65536, 4096), gen, device, 1e-3)
    x = _randn((65536, 7168), gen, device)
    return dy, x, sizes


def c5_sizes(seed=0):
    return zipf_sizes(131072, 32, 1.0, seed)


def topk_routing(tokens: int, experts: int, topk: int, s: float, seed: int = 0):
    """Top-k routing decisions of a MoE router: for every token, topk distinct
    experts drawn with Zipf(s) preference p_i ~ 1/i^s (Gumbel top-k, i.e.
    sampling without replacement), and softmax-normalised scores over them.
    Returns (expert_idx int32 [tokens, topk], scores float32 [tokens, topk])."""
    rng = np.random.default_rng(seed)
    logp = -s * np.log(np.arange(1, experts + 1, dtype=np.float64))
    keys = logp[None, :] + rng.gumbel(size=(tokens, experts))
    idx = np.argsort(-keys, axis=1)[:, :topk].astype(np.int32)
    logits = rng.standard_normal((tokens, topk))
    w = np.exp(logits - logits.max(axis=1, keepdims=True))
    return idx, (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


def c5_routing(seed=0):
    """C5's 131072 routed tokens as 16384 tokens x top-8 over 32 experts, Zipf(1.0)."""
    return topk_routing(16384, 32, 8, 1.0, seed)


def gemm_flops(tokens: int, n: int, k: int) -> int:
    """Algorithmic FLOPs of a grouped GEMM: 2 * M_total * N * K (fused_fwd.py:341)."""
    return 2 * int(tokens) * int(n) * int(k)
