"""Closed-form probes of the DiT's time and text embeddings (causal_model.py:519-525,840-855).

One-hot weights (a single 1 in each output row, at an input column picked by a seeded
permutation) and zero biases make each linear a column gather, exact in any summation order,
so the embeddings reduce to their activations applied to chosen inputs:

* time: s = bf16(sinusoid(t)) (cos half, then sin half); the time embedding
  Linear -> SiLU -> Linear gives h_o = bf16(silu(s[j1(o)])) and e_o = h[j2(o)]; the time
  projection SiLU -> Linear gives e0_o = bf16(silu(e[j3(o)]));
* text: Linear -> GELU(tanh) -> Linear over the context padded with zero rows to 512 gives
  h_o = bf16(gelu_tanh(ctx[:, j(o)])) (0 on the padding rows) and out_o = bf16(h[k(o)] + b2_o),
  so the padding rows read back the second bias exactly.

The activations are evaluated from their definitions in float64 (silu(x) = x / (1 + e^-x),
gelu_tanh(x) = x / 2 * (1 + tanh(sqrt(2 / pi) * (x + 0.044715 x^3)))) and rounded to bf16; an
fp32 or hardware evaluation may land one bf16 ulp away near a rounding boundary, so a probe
allows one ulp.  A dropped or exchanged activation moves most elements by many ulps
(``time_alternatives`` / ``text_alternatives``).
"""

from __future__ import annotations

import dataclasses
import math

import torch

BF16 = torch.bfloat16
FREQ = 256
TEXT_DIM = 4096
TEXT_LEN = 512


def _one_hot(rows: int, cols: int, pick: torch.Tensor) -> torch.Tensor:
    w = torch.zeros((rows, cols), dtype=BF16)
    w[torch.arange(rows), pick] = 1
    return w


def _pick(n: int, cols: int, g) -> torch.Tensor:
    """n column indices < cols, a seeded permutation repeated as needed."""
    reps = -(-n // cols)
    return torch.cat([torch.randperm(cols, generator=g) for _ in range(reps)])[:n]


def silu64(x: torch.Tensor) -> torch.Tensor:
    x = x.double()
    return x / (1 + torch.exp(-x))


def gelu_tanh64(x: torch.Tensor) -> torch.Tensor:
    x = x.double()
    return 0.5 * x * (1 + torch.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))


def sinusoid(t: float, frames: int) -> torch.Tensor:
    """cos(t w_i) for i < 128, then sin(t w_i), w_i = 10000^(-i/128) (model.py:15-26), float64 [frames, 256]."""
    i = torch.arange(FREQ // 2, dtype=torch.float64)
    a = float(t) * torch.pow(torch.tensor(10000.0, dtype=torch.float64), -i / (FREQ // 2))
    return torch.cat([torch.cos(a), torch.sin(a)]).unsqueeze(0).expand(frames, FREQ)


def time_probe(params, seed: int = 0):
    """params with one-hot time weights and zero biases, and the column picks (j1, j2, j3)."""
    dim = params.dim
    g = torch.Generator().manual_seed(300 + seed)
    j1, j2, j3 = _pick(dim, FREQ, g), _pick(dim, dim, g), _pick(6 * dim, dim, g)
    p = dataclasses.replace(
        params, time1_w=_one_hot(dim, FREQ, j1), time1_b=torch.zeros(dim, dtype=BF16),
        time2_w=_one_hot(dim, dim, j2), time2_b=torch.zeros(dim, dtype=BF16),
        proj_w=_one_hot(6 * dim, dim, j3), proj_b=torch.zeros(6 * dim, dtype=BF16))
    return p, (j1, j2, j3)


def time_closed_form(t: float, frames: int, picks, silu_time=True, silu_proj=True):
    """(e [F, dim], e0 [F, 6, dim]) bf16; ``silu_time`` / ``silu_proj`` False drop one SiLU."""
    j1, j2, j3 = picks
    s = sinusoid(t, frames).to(BF16)
    pre = s[:, j1]
    h = (silu64(pre) if silu_time else pre.double()).to(BF16)
    e = h[:, j2]
    pe = e[:, j3]
    e0 = (silu64(pe) if silu_proj else pe.double()).to(BF16)
    return e, e0.view(frames, 6, -1)


def time_alternatives(t: float, frames: int, picks) -> dict:
    return {"no SiLU after the first time linear": time_closed_form(t, frames, picks, silu_time=False),
            "no SiLU before the time projection": time_closed_form(t, frames, picks, silu_proj=False)}


def text_probe(params, context_len: int = 300, seed: int = 0):
    """params with one-hot text weights, zero first bias and a random second bias; the context
    [context_len, 4096] bf16 (~N(0, 1.5)); and the column picks (j, k)."""
    dim = params.dim
    g = torch.Generator().manual_seed(400 + seed)
    j, k = _pick(dim, TEXT_DIM, g), _pick(dim, dim, g)
    b2 = (torch.randn(dim, generator=g) * 0.05).to(BF16)
    ctx = (torch.randn((context_len, TEXT_DIM), generator=g) * 1.5).to(BF16)
    p = dataclasses.replace(params, text1_w=_one_hot(dim, TEXT_DIM, j), text1_b=torch.zeros(dim, dtype=BF16),
                            text2_w=_one_hot(dim, dim, k), text2_b=b2)
    return p, ctx, (j, k)


def text_closed_form(ctx: torch.Tensor, b2: torch.Tensor, picks, gelu=True):
    """[512, dim] bf16 text embedding of the probe; ``gelu`` False drops the GELU."""
    j, k = picks
    pad = torch.zeros((TEXT_LEN - ctx.shape[0], ctx.shape[1]), dtype=BF16)
    x = torch.cat([ctx, pad])[:, j]
    h = (gelu_tanh64(x) if gelu else x.double()).to(BF16)
    return (h[:, k].double() + b2.double()).to(BF16)


def text_alternatives(ctx, b2, picks) -> dict:
    j, k = picks
    pad = torch.zeros((TEXT_LEN - ctx.shape[0], ctx.shape[1]), dtype=BF16)
    x = torch.cat([ctx, pad])[:, j]
    silu_form = (silu64(x).to(BF16)[:, k].double() + b2.double()).to(BF16)
    return {"no GELU": text_closed_form(ctx, b2, picks, gelu=False), "SiLU in place of GELU": silu_form}


def ulp(x: torch.Tensor) -> torch.Tensor:
    return torch.pow(2.0, torch.floor(torch.log2(x.double().abs().clamp(min=2.0 ** -100))) - 7)


def within_one_ulp(got: torch.Tensor, want: torch.Tensor) -> bool:
    return bool(((got.double() - want.double()).abs() <= ulp(want) + 1e-30).all())


def far_fraction(alt: torch.Tensor, want: torch.Tensor) -> float:
    """Fraction of elements where ``alt`` is more than one ulp from ``want``."""
    return ((alt.double() - want.double()).abs() > ulp(want) + 1e-30).double().mean().item()
