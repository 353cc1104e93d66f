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
