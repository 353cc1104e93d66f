"""Attention oracle (torch CPU, fp32).

The reference's wavefront attention is non-causal over the assembled
context (wave_rt/runtime/backend.py:141-148, ``causal=False``); its SDPA
fallback is naive_rt/rolling_forcing/wan/modules/attention.py:75-89
(transpose to [B, N, L, C], ``scaled_dot_product_attention``, transpose
back).  Over FP8 pages the context is first unpacked to bf16 K/V
(oracle.kv.unpack, the reference's dequant of common.py:161-164) and then
attended in fp32.
"""

from __future__ import annotations

import math
from typing import Sequence

import torch

from . import kv as okv


def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float | None = None) -> torch.Tensor:
    """q [Lq, H, D], k/v [Lk, H, D] -> fp32 [Lq, H, D]; softmax(q k^T * scale) v per head."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    H = q.shape[1]
    # the score tensor of a whole 14B context is tens of GB: heads go in groups of at most 2^28 scores
    group = max(1, min(H, (1 << 28) // max(1, q.shape[0] * k.shape[0])))
    outs = []
    for h0 in range(0, H, group):
        sl = slice(h0, h0 + group)
        qh = q[:, sl].float().transpose(0, 1)  # [h, Lq, D]
        kh = k[:, sl].float().transpose(0, 1)
        vh = v[:, sl].float().transpose(0, 1)
        s = torch.matmul(qh, kh.transpose(1, 2)) * scale
        pr = torch.softmax(s, dim=-1)
        outs.append(torch.matmul(pr, vh).transpose(0, 1))
    return outs[0] if len(outs) == 1 else torch.cat(outs, dim=1)


def paged_fp8(q, k_pool, v_pool, table: Sequence[int], n_kv: int, page_tokens: int, scale=None) -> torch.Tensor:
    """q [Lq, H, D] bf16 against FP8 pools ((codes, scales) pairs) -> fp32 [Lq, H, D]."""
    k = okv.unpack(table, n_kv, page_tokens, *k_pool)
    v = okv.unpack(table, n_kv, page_tokens, *v_pool)
    return sdpa(q, k, v, scale)


def quantize_q_rows(q: torch.Tensor):
    """e4m3 quantization of each query row (per head) with a power-of-two scale: s_q = 2^e, the smallest power
    of two with amax|q| <= 448 s_q (1 for an all-zero row), and codes e4m3(q / s_q), where the division by a power
    of two is exact, so each code is the e4m3 rounding (to nearest, ties to even) of q 2^-e itself.
    q [Lq, H, D] bf16 -> (fp32 decoded codes [Lq, H, D], s_q [Lq, H])."""
    qf = q.float()
    amax = qf.abs().amax(dim=-1)
    mant, expo = torch.frexp(amax.double())            # amax = mant 2^expo, mant in [0.5, 1)
    e = torch.where(mant <= 0.875, expo - 9, expo - 8)  # 448 = 0.875 2^9
    e = torch.where(amax > 0, e, torch.zeros_like(e)).clamp(-127, 127)
    s_q = torch.pow(2.0, e.double()).float()
    codes = torch.ldexp(qf.double(), -e[..., None].double()).clamp(-448.0, 448.0).float().to(okv.FP8).float()
    return codes, s_q


def paged_fp8_qk8(q, k_pool, v_pool, table: Sequence[int], n_kv: int, page_tokens: int, scale=None) -> torch.Tensor:
    """The quantized-QK form of :func:`paged_fp8` (the counterpart of the reference's SageAttention backend,
    wave_rt/runtime/backend.py:57-62,144-146, which quantizes Q and K before QK^T): scores
    (sum_d code_q code_k) * s_q * s_k * scale over the e4m3 K codes of the pages and the per-row e4m3 queries of
    :func:`quantize_q_rows`, softmax in float64, V the pages' bf16 dequantization.  -> fp32 [Lq, H, D]."""
    kc, ks = okv.gather(table, n_kv, page_tokens, *k_pool)
    v = okv.unpack(table, n_kv, page_tokens, *v_pool)
    return sdpa_qk8(q, kc, ks, v, scale)


def sdpa_qk8(q, k_codes, k_scales, v, scale=None) -> torch.Tensor:
    """The quantized-QK attention over dense operands: q [Lq, H, D] bf16, K as e4m3 codes [Lk, H, D] (uint8)
    with scales [Lk, H], v [Lk, H, D] -> fp32 [Lq, H, D] (the body of :func:`paged_fp8_qk8`)."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    qc, sq = quantize_q_rows(q)
    kcf = k_codes.view(okv.FP8).float().double()                  # [Lk, H, D]
    out = []
    for h in range(q.shape[1]):
        s = (qc[:, h].double() @ kcf[:, h].T) * sq[:, h, None].double() * k_scales[:, h][None, :].double() * scale
        out.append(torch.softmax(s, dim=-1) @ v[:, h].double())
    return torch.stack(out, dim=1).float()
