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


LOG2E = 1.4426950408889634
TILE_KEYS = 64      # keys per step of the fp8-PV form
RESCALE_TAU = 8.0   # lazy-rescale threshold (log2 units)


def _f32(x: torch.Tensor) -> torch.Tensor:
    """Round float64 values to fp32 (kept as float64)."""
    return x.float().double()


def pv8_exponent(mx: torch.Tensor) -> torch.Tensor:
    """E for weights of maximum mx >= 0: the smallest power of two with mx <= 448 2^E (the queries' rule of
    :func:`quantize_q_rows`), 0 for mx = 0, clamped to [-126, 127]."""
    mant, expo = torch.frexp(mx)
    e = torch.where(mant <= 0.875, expo - 9, expo - 8)
    return torch.where(mx > 0, e, torch.zeros_like(e)).clamp(-126, 127)


def paged_fp8_qkpv8(q, k_pool, v_pool, table: Sequence[int], n_kv: int, page_tokens: int, scale=None,
                    round_p: bool = True, margin_eps: float | None = None):
    """The quantized-QK form with the P.V product on e4m3 weights (the counterpart of the fp8 P.V product of the
    reference's SageAttention backend, wave_rt/runtime/backend.py:57-62,144-146) over the pages' K and V codes
    -> fp32 [Lq, H, D] (and the rounding margin with ``margin_eps``); see :func:`sdpa_qkpv8`."""
    kc, ks = okv.gather(table, n_kv, page_tokens, *k_pool)
    vc, vs = okv.gather(table, n_kv, page_tokens, *v_pool)
    return sdpa_qkpv8(q, kc, ks, vc, vs, scale, round_p, margin_eps)


def _e4m3_step(y: torch.Tensor) -> torch.Tensor:
    """The spacing of the e4m3 values around y >= 0: 2^(floor(log2 y) - 3) in the normal range, 2^-9 below it."""
    return torch.pow(2.0, torch.floor(torch.log2(y.clamp(min=2.0 ** -6))) - 3)


def sdpa_qkpv8(q, k_codes, k_scales, v_codes, v_scales, scale=None, round_p: bool = True,
               margin_eps: float | None = None):
    """Attention with e4m3 queries and e4m3 weights over K/V codes [Lk, H, D] (uint8) with scales [Lk, H].

    The weights are formed as the HIP kernel forms them, step by step, so that their e4m3 rounding sees the same
    values: keys in tiles of 64, each query with its own lazy maximum.  Scores
    s = (sum_d code_q code_k) s_q with u_k = fp32(s_k * fp32(scale * log2 e)); per tile and query the bound
    max(s) * max(0, max u) over each half of the tile's keys (the keys whose index has bit 2 clear / set; 0 when
    the half's max(s) < 0), and a query whose bound exceeds its threshold takes m = max(m, max_k fp32(s u_k))
    with O and l scaled by 2^(m_old - m) and threshold m + 8.  Then
    p_k = 2^fp32(s u_k - m), l += p_k, w_k = fp32(p_k s_v,k); 2^E from the tile's max w (:func:`pv8_exponent`);
    O += sum_k e4m3(w_k / 2^E) 2^E code_v,k.  Out: O / l.  With ``round_p`` False the weights are not rounded,
    which leaves the quantized-QK attention of :func:`sdpa_qk8` over the dequantized V.

    A weight whose w_k / 2^E lies within a relative ``margin_eps`` of the midpoint between two e4m3 values may
    round to either of them in an implementation whose fp32 scores or exponentials differ in the last bits;
    with ``margin_eps`` the call also returns, per output element, the sum over such weights of
    step * 2^E * |code_v| / l (what rounding the other way would move it by): (out, margin).
    """
    Lq, H, D = q.shape
    n_kv = k_codes.shape[0]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    c32 = float(torch.tensor(scale, dtype=torch.float32) * torch.tensor(LOG2E, dtype=torch.float32))
    qc, sq = quantize_q_rows(q)
    out = torch.zeros((Lq, H, D), dtype=torch.float64)
    margin = torch.zeros_like(out)
    if n_kv == 0:
        return (out.float(), margin.float()) if margin_eps is not None else out.float()
    n_tiles = -(-n_kv // TILE_KEYS)
    Kp = n_tiles * TILE_KEYS
    half = ((torch.arange(TILE_KEYS) >> 2) & 1).bool()              # bit 2 of the key index in its tile
    kcf = k_codes.view(okv.FP8).float().double()
    vcf = v_codes.view(okv.FP8).float().double()
    for h in range(H):
        s = torch.full((Lq, Kp), -math.inf, dtype=torch.float64)
        s[:, :n_kv] = _f32((qc[:, h].double() @ kcf[:, h].T) * sq[:, h, None].double())
        u = torch.ones(Kp, dtype=torch.float64)
        u[:n_kv] = _f32(k_scales[:, h].float().double() * c32)
        sv = torch.zeros(Kp, dtype=torch.float64)
        sv[:n_kv] = v_scales[:, h].float().double()
        vh = torch.zeros((Kp, D), dtype=torch.float64)
        vh[:n_kv] = vcf[:, h]
        m = torch.full((Lq,), -math.inf, dtype=torch.float64)
        thr = torch.full((Lq,), -math.inf, dtype=torch.float64)
        o = torch.zeros((Lq, D), dtype=torch.float64)
        amb = torch.zeros((Lq, D), dtype=torch.float64)
        l = torch.zeros(Lq, dtype=torch.float64)
        for t in range(n_tiles):
            ks = slice(t * TILE_KEYS, (t + 1) * TILE_KEYS)
            st, ut = s[:, ks], u[ks]
            bound = None
            for hm in (~half, half):
                mt = st[:, hm].amax(dim=1)
                um = max(0.0, float(ut[hm].max()))
                b = torch.where(mt >= 0, _f32(mt * um), torch.zeros_like(mt))
                bound = b if bound is None else torch.maximum(bound, b)
            fire = bound > thr
            if bool(fire.any()):
                ex = _f32(st * ut[None, :]).amax(dim=1)
                m_new = torch.maximum(m, ex)
                alpha = torch.where(m == -math.inf, torch.zeros_like(m), _f32(torch.exp2(_f32(m - m_new))))
                alpha = torch.where(fire, alpha, torch.ones_like(alpha))
                o *= alpha[:, None]
                amb *= alpha[:, None]
                l *= alpha
                m = torch.where(fire, m_new, m)
                thr = torch.where(fire, _f32(m_new + RESCALE_TAU), thr)
            neg = torch.where(m == -math.inf, torch.zeros_like(m), -m)
            p = _f32(torch.exp2(_f32(st * ut[None, :] + neg[:, None])))
            l += p.sum(dim=1)
            w = _f32(p * sv[ks][None, :])
            if round_p:
                sc = torch.pow(2.0, pv8_exponent(w.amax(dim=1)).double())[:, None]
                y = w / sc
                if margin_eps is not None:
                    step = _e4m3_step(y)
                    near = ((y - (torch.floor(y / step) * step + step / 2)).abs() <= margin_eps * y) & (y > 0)
                    amb += (near.double() * step * sc) @ vh[ks].abs()
                w = y.float().to(okv.FP8).double() * sc
            o += w @ vh[ks]
        res = torch.where(l[:, None] > 0, o / l[:, None], torch.zeros_like(o))
        out[:, h] = res
        margin[:, h] = torch.where(l[:, None] > 0, amb / l[:, None], torch.zeros_like(amb))
    return (out.float(), margin.float()) if margin_eps is not None else out.float()
