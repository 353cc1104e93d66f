"""Wan attention block oracle (torch CPU) on the quantized path.

Restates CausalWanAttentionBlock.forward
(naive_rt/rolling_forcing/wan/modules/causal_model.py:349-402) in the dtypes
the reference runs it in (the model is bf16; the autocast blocks are
commented out, causal_model.py:375,385,396):

* e = (modulation + e).chunk(6) in bf16 (:376);
* WanLayerNorm (model.py:89-99), WanRMSNorm (model.py:70-86);
* modulation and gated residuals as bf16 tensor ops (:381,386,390,393-398);
* RoPE as causal_rope_apply (:27-55: float64 complex rotation, rounded to
  bf16) with the 22/21/21 frame/height/width split;
* every linear as the int8 W8A8 oracle (oracle.linear, scope ``all``), the
  FFN activation GELU(tanh) on the bf16 fc_in output (:342-344);
* self-attention over the FP8 paged context (oracle.attention.paged_fp8,
  own chunk packed into its pages first), cross-attention over the text K/V
  (model.py:159-194, k = norm_k(k(context)), v = v(context)); attention
  outputs are rounded to bf16 like the reference's attention kernels.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import attention as oat
from . import kv as okv
from . import linear as olin

EPS = 1e-6


def layer_norm(x, w=None, b=None):
    return F.layer_norm(x, (x.shape[-1],), w, b, EPS)


def rms_norm(x, w):
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + EPS)).type_as(x) * w


def rope_angles(frames, height, width, start_frame, head_dim=128, theta=10000.0):
    """float64 [T, head_dim/2] angles of causal_rope_apply's frequency table."""
    c = head_dim // 2
    dims = [c - 2 * (c // 3), c // 3, c // 3]

    def rope_params(max_len, dim):  # model.py:29-36, angles only
        return torch.outer(torch.arange(max_len, dtype=torch.float64),
                           1.0 / torch.pow(torch.tensor(theta, dtype=torch.float64),
                                           torch.arange(0, dim, 2, dtype=torch.float64).div(dim)))

    ft = rope_params(1024, 2 * dims[0])[start_frame:start_frame + frames]
    fh = rope_params(1024, 2 * dims[1])[:height]
    fw = rope_params(1024, 2 * dims[2])[:width]
    a = torch.cat([
        ft.view(frames, 1, 1, -1).expand(frames, height, width, -1),
        fh.view(1, height, 1, -1).expand(frames, height, width, -1),
        fw.view(1, 1, width, -1).expand(frames, height, width, -1),
    ], dim=-1)
    return a.reshape(frames * height * width, c)


def rope_apply(x, angles):
    """x [T, H, D] bf16 -> bf16, pairs (2i, 2i+1) rotated by angles[T, i] in float64."""
    T, H, D = x.shape
    xc = torch.view_as_complex(x.to(torch.float64).reshape(T, H, D // 2, 2))
    rot = torch.polar(torch.ones_like(angles), angles).view(T, 1, D // 2)
    return torch.view_as_real(xc * rot).flatten(2).to(x.dtype)


def rope_apply_table(x, cos, sin):
    """x [T, H, D] bf16 rotated by fp32 tables cos/sin [T, D/2] -> bf16.

    The table form of the same rotation, as the exchange applies it with
    SGLang's precomputed cos/sin (_anchor_rope / _apply_rotary_emb with
    is_neox_style=False, wave_rt/denoiser/exchange/common.py:45-91,
    backend.py:119-121): pair (a, b) = (x[2i], x[2i+1]) becomes
    (a*c - b*s, a*s + b*c), each product, difference and sum an fp32 operation,
    then rounded once to bf16.
    """
    T, H, D = x.shape
    xf = x.float().reshape(T, H, D // 2, 2)
    a, b = xf[..., 0], xf[..., 1]
    c = cos.float().view(T, 1, D // 2)
    s = sin.float().view(T, 1, D // 2)
    out = torch.stack((a * c - b * s, a * s + b * c), dim=-1)
    return out.reshape(T, H, D).to(torch.bfloat16)


def block_forward(p, x, e, grid, start_frame, pool_k, pool_v, context_table, own_table, n_context, page_tokens,
                  text_k, text_v, heads, return_unroped_k=False, paged_attn=None):
    """One block on the CPU.

    p: waveforcing_amd.block.BlockParams (CPU bf16); x [T, dim] bf16;
    e [F, 6, dim] bf16; grid = (frames, height, width) of the chunk;
    pool_k / pool_v: (codes, scales) CPU pools holding the prior context, into
    which this chunk's K/V are packed at own_table (modified in place);
    text_k / text_v [L, H, D] bf16.  Returns the new x, and with
    ``return_unroped_k`` also the chunk's normalized, un-rotated K [T, H, D]
    (the exchange's unroped_key).  ``paged_attn`` replaces the self-attention
    over the pages (default :func:`oracle.attention.paged_fp8`; the reference
    swaps its attention function the same way, backend.py:141-148).
    """
    T, dim = x.shape
    frames, height, width = grid
    hd = dim // heads
    ft = T // frames
    es = (p.modulation[0].unsqueeze(0) + e)  # [F, 6, dim], bf16

    def per_frame(t, k):  # t [T, dim] * / + e[:, k] broadcast per frame
        return es[:, k].repeat_interleave(ft, dim=0)

    def lin(t, w, b, gelu=False):
        return olin.i8_linear(t, w, b, gelu=gelu)

    # self-attention
    a = layer_norm(x)
    a = a * (1 + per_frame(a, 1)) + per_frame(a, 0)
    q = rms_norm(lin(a, p.q_w, p.q_b), p.norm_q).view(T, heads, hd)
    ku = rms_norm(lin(a, p.k_w, p.k_b), p.norm_k).view(T, heads, hd)
    v = lin(a, p.v_w, p.v_b).view(T, heads, hd)
    ang = rope_angles(frames, height, width, start_frame, hd)
    q = rope_apply(q, ang)
    k = rope_apply(ku, ang)
    okv.pack(k, own_table, page_tokens, *pool_k)
    okv.pack(v, own_table, page_tokens, *pool_v)
    y = (paged_attn or oat.paged_fp8)(q, pool_k, pool_v, context_table, n_context, page_tokens).to(torch.bfloat16)
    y = lin(y.reshape(T, dim), p.o_w, p.o_b)
    x = x + y * per_frame(y, 2)

    # cross-attention
    c = layer_norm(x, p.norm3_w, p.norm3_b)
    cq = rms_norm(lin(c, p.cq_w, p.cq_b), p.cnorm_q).view(T, heads, hd)
    y = oat.sdpa(cq, text_k, text_v).to(torch.bfloat16)
    x = x + lin(y.reshape(T, dim), p.co_w, p.co_b)

    # FFN
    h = layer_norm(x)
    h = h * (1 + per_frame(h, 4)) + per_frame(h, 3)
    f = lin(h, p.fc_in_w, p.fc_in_b, gelu=True)
    y = lin(f, p.fc_out_w, p.fc_out_b)
    x = x + y * per_frame(y, 5)
    return (x, ku) if return_unroped_k else x


def text_kv(p, context, heads):
    """Cross-attention K/V of the text context (model.py:177-178)."""
    L, dim = context.shape
    k = rms_norm(olin.i8_linear(context, p.ck_w, p.ck_b), p.cnorm_k).view(L, heads, dim // heads)
    v = olin.i8_linear(context, p.cv_w, p.cv_b).view(L, heads, dim // heads)
    return k, v
