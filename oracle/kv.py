"""FP8 KV oracle: per-(token, head) quantization, page scatter, gather-dequant.

Follows the reference's FP8 KV quantization, wave_rt/denoiser/exchange/
common.py:145-150, with the amax taken over the head dimension of each
(token, head) row in place of the whole tensor:

    scale = (kv.abs().amax(-1, keepdim=True) / 448.0).clamp(min=1e-8).to(float32)
            -- bf16 arithmetic before the final cast, as in the reference
    codes = (kv / scale).clamp(-448, 448).to(float8_e4m3fn)
            -- kv / scale divides in fp32 because the scale is a dimensioned
               fp32 tensor; the +-448 clamp is the workload's stated clamp

and its dequant, common.py:161-164 (``codes.to(bf16) * scale`` -> fp32), here
rounded once to bf16.  Pages follow wave_rt/denoiser/exchange/paged.py:137
(slot rows of ``T`` tokens, ``[H, D]`` per token) with an arbitrary page table.
"""

from __future__ import annotations

from typing import Sequence

import torch

FP8 = torch.float8_e4m3fn
E4M3_MAX = 448.0


def quantize_rows(kv: torch.Tensor):
    """kv bf16 [..., D] -> (codes uint8 [..., D], scales fp32 [...])."""
    assert kv.dtype == torch.bfloat16
    scale = (kv.abs().amax(dim=-1, keepdim=True) / E4M3_MAX).clamp(min=1e-8).to(torch.float32)
    q = (kv / scale).clamp(-E4M3_MAX, E4M3_MAX)
    codes = q.to(FP8).view(torch.uint8)
    return codes, scale.squeeze(-1)


def dequantize_rows(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """codes uint8 [..., D], scales fp32 [...] -> bf16 [..., D]."""
    return (codes.view(FP8).to(torch.bfloat16) * scales.unsqueeze(-1)).to(torch.bfloat16)


def new_pool(pool_pages: int, page_tokens: int, n_heads: int, head_dim: int):
    """Zeroed CPU pool (codes [P, page, H, D] uint8, scales [P, H, page] fp32)."""
    return (
        torch.zeros((pool_pages, page_tokens, n_heads, head_dim), dtype=torch.uint8),
        torch.zeros((pool_pages, n_heads, page_tokens), dtype=torch.float32),
    )


def pack(kv: torch.Tensor, table: Sequence[int], page_tokens: int, codes_pool, scales_pool) -> None:
    """Quantize kv [T, H, D] and scatter into the pool pages listed in ``table`` (in place)."""
    T = kv.shape[0]
    codes, scales = quantize_rows(kv)
    for lp in range(-(-T // page_tokens)):
        page = int(table[lp])
        t0, t1 = lp * page_tokens, min(T, (lp + 1) * page_tokens)
        if page < 0 or page >= codes_pool.shape[0]:
            continue
        codes_pool[page, : t1 - t0] = codes[t0:t1]
        scales_pool[page, :, : t1 - t0] = scales[t0:t1].transpose(0, 1)


def gather(table: Sequence[int], n_tokens: int, page_tokens: int, codes_pool, scales_pool):
    """Logical tokens [0, n_tokens) of the pool -> (codes [T, H, D], scales [T, H])."""
    cs, ss = [], []
    for lp in range(-(-n_tokens // page_tokens)):
        page = int(table[lp])
        n = min(page_tokens, n_tokens - lp * page_tokens)
        cs.append(codes_pool[page, :n])
        ss.append(scales_pool[page, :, :n].transpose(0, 1))
    return torch.cat(cs, 0), torch.cat(ss, 0)


def unpack(table: Sequence[int], n_tokens: int, page_tokens: int, codes_pool, scales_pool) -> torch.Tensor:
    """Gather + dequantize to bf16 [T, H, D]."""
    codes, scales = gather(table, n_tokens, page_tokens, codes_pool, scales_pool)
    return dequantize_rows(codes, scales)


# ------------------------------------------------------------ per tensor
def quantize_tensor(kv: torch.Tensor):
    """The reference's per-tensor FP8 KV quantization, wave_rt/denoiser/exchange/common.py:145-150, in its
    own torch dtypes: the bf16 amax / 448 stays bf16, the clamp floor is bf16(1e-8), the scale is then cast to
    fp32 (0-dim); bf16 kv divided by that 0-dim fp32 scale stays bf16 (the quotient is rounded to bf16) and is
    cast to e4m3fn.  kv bf16 [...] -> (codes uint8 [...], scale fp32 [1])."""
    assert kv.dtype == torch.bfloat16
    scale = (kv.abs().amax() / E4M3_MAX).clamp(min=1e-8).to(torch.float32)
    codes = (kv / scale).to(FP8).view(torch.uint8)
    return codes, scale.reshape(1)


def dequantize_tensor(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """common.py:161-164: ``codes.view(e4m3).to(bf16) * scale`` with the 1-element fp32 scale -> fp32."""
    return codes.view(FP8).to(torch.bfloat16) * scale
