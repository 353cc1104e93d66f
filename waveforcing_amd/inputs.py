"""Seeded synthetic inputs of the benchmark workloads (generated on the CPU).

Every tensor comes from its own ``torch.Generator`` with a fixed seed, so the
GPU run and the CPU baseline see identical values.

Workloads (Wan2.1 shapes; a chunk is 3 latent frames = 4680 tokens):
  linear_1p3b   X bf16 [4680, 1536] ~ N(0,1) with 1% of channels (15, chosen
                by randperm(1536, seed 3)) scaled x20; W bf16 [1536, 1536]
                ~ N(0, 0.02) (seed 1); bias bf16 ~ N(0, 0.01) (seed 2).
  kv_layer      K, V bf16 [4680, 12, 128] ~ N(0,1) where 8 of the 128 head-dim
                indices of every head carry Student-t(3) values
                Z / sqrt(chi2_3 / 3) (heavy-tailed outliers).
"""

from __future__ import annotations

import torch


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def outlier_activations(m: int, k: int, seed: int = 0, chan_seed: int = 3, frac: float = 0.01,
                        gain: float = 20.0) -> torch.Tensor:
    """bf16 [m, k] ~ N(0,1) with round(frac*k) channels scaled by ``gain``."""
    x = torch.randn((m, k), generator=_gen(seed), dtype=torch.float32)
    n_out = max(1, round(frac * k))
    chans = torch.randperm(k, generator=_gen(chan_seed))[:n_out]
    x[:, chans] *= gain
    return x.to(torch.bfloat16)


def linear_weights(n: int, k: int, w_seed: int = 1, b_seed: int = 2, w_std: float = 0.02,
                   b_std: float = 0.01):
    """(W bf16 [n, k] ~ N(0, w_std), bias bf16 [n] ~ N(0, b_std))."""
    w = (torch.randn((n, k), generator=_gen(w_seed)) * w_std).to(torch.bfloat16)
    b = (torch.randn((n,), generator=_gen(b_seed)) * b_std).to(torch.bfloat16)
    return w, b


def linear_1p3b():
    """The single W8A8 linear at Wan-1.3B shape: (x, w, bias)."""
    x = outlier_activations(4680, 1536, seed=0, chan_seed=3)
    w, b = linear_weights(1536, 1536, w_seed=1, b_seed=2)
    return x, w, b


def heavy_tailed_kv(tokens: int, heads: int, head_dim: int, seed: int, n_heavy: int = 8) -> torch.Tensor:
    """bf16 [tokens, heads, head_dim] ~ N(0,1), with ``n_heavy`` Student-t(3) dims per head."""
    g = _gen(seed)
    x = torch.randn((tokens, heads, head_dim), generator=g)
    for h in range(heads):
        dims = torch.randperm(head_dim, generator=g)[:n_heavy]
        z = torch.randn((tokens, n_heavy), generator=g)
        chi2 = torch.randn((tokens, n_heavy, 3), generator=g).pow(2).sum(-1)
        x[:, h, dims] = z / torch.sqrt(chi2 / 3.0)
    return x.to(torch.bfloat16)


def kv_layer(layer: int, tokens: int = 4680, heads: int = 12, head_dim: int = 128, seed: int = 100):
    """(K, V) of one layer of the FP8 KV workload; seeds 100 + 2*layer (+1 for V)."""
    k = heavy_tailed_kv(tokens, heads, head_dim, seed + 2 * layer)
    v = heavy_tailed_kv(tokens, heads, head_dim, seed + 2 * layer + 1)
    return k, v


def page_table(n_pages: int, pool_pages: int, seed: int = 7) -> list[int]:
    """Seeded random physical page ids (distinct) for ``n_pages`` logical pages."""
    if n_pages > pool_pages:
        raise ValueError("pool too small")
    return torch.randperm(pool_pages, generator=_gen(seed))[:n_pages].tolist()
