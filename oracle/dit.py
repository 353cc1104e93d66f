"""The Wan DiT's layers around the blocks (torch CPU), test infrastructure only: what
waveforcing_amd.dit is tested against.

Restates, in the dtypes the reference runs them (a bf16 model; the autocast
blocks are commented out, causal_model.py:841,871):

* the patch embedding, nn.Conv3d(16, dim, kernel = stride = (1, 2, 2))
  (causal_model.py:517-518), then ``flatten(2).transpose(1, 2)``
  (:826-830): written as the patch gather + a linear over the weight viewed
  [dim, 64], pinned against F.conv3d by the tests;
* sinusoidal_embedding_1d (model.py:15-26, float64), the time embedding
  Linear -> SiLU -> Linear and the time projection SiLU -> Linear(dim, 6 dim)
  (causal_model.py:522-525,840-844), the text embedding
  Linear(4096, dim) -> GELU(tanh) -> Linear(dim, dim) over the context padded
  to 512 tokens (:519-521,848-855);
* the head, LayerNorm (no affine) * (1 + e[1]) + e[0] with
  e = head.modulation + time embedding, then Linear(dim, 64)
  (CausalHead, :406-433);
* unpatchify, 'fhwpqrc->cfphqwr' (:1080-1103);
* the flow -> x0 conversion x0 = xt - sigma * flow in float64 with sigma at
  the nearest timestep (wan_wrapper.py:169-193), cast back to bf16.

Every bf16 nn.Linear is evaluated as an fp32 product of the bf16 operands with
the bias added in fp32 and one rounding to bf16; every activation module acts
on bf16 values in fp32 and rounds to bf16.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

BF16 = torch.bfloat16
EPS = 1e-6


def linear(x, w, b=None, act_out=None, silu_in=False):
    """bf16 nn.Linear (fp32 accumulation, fp32 bias, one rounding), with an optional SiLU on the input
    (an nn.SiLU module before it) and an optional SiLU / GELU(tanh) module after it."""
    xf = x.float()
    if silu_in:
        xf = F.silu(xf).to(BF16).float()
    y = F.linear(xf, w.float(), None if b is None else b.float()).to(BF16)
    if act_out == "silu":
        y = F.silu(y.float()).to(BF16)
    elif act_out == "gelu":
        y = F.gelu(y.float(), approximate="tanh").to(BF16)
    return y


def patchify(latent):
    """latent [C, F, H, W] -> patches [F*(H/2)*(W/2), 4C] in the Conv3d weight's (c, kh, kw) order."""
    C, Fr, H, W = latent.shape
    p = latent.reshape(C, Fr, H // 2, 2, W // 2, 2).permute(1, 2, 4, 0, 3, 5)
    return p.reshape(Fr * (H // 2) * (W // 2), C * 4)


def patch_embed(latent, w, b):
    """latent [C, F, H, W] bf16, Conv3d weight [dim, C, 1, 2, 2] -> tokens [T, dim] bf16."""
    return linear(patchify(latent), w.reshape(w.shape[0], -1), b)


def sinusoidal_embedding_1d(dim, position):
    """model.py:15-26: float64 [len(position), dim], cos half then sin half."""
    half = dim // 2
    pos = position.to(torch.float64)
    sinusoid = torch.outer(pos, torch.pow(10000, -torch.arange(half).to(pos).div(half)))
    return torch.cat([torch.cos(sinusoid), torch.sin(sinusoid)], dim=1)


def time_embed(p, t_frames, freq_dim=256):
    """t_frames [F] -> (e [F, dim], e0 [F, 6, dim]) bf16."""
    s = sinusoidal_embedding_1d(freq_dim, t_frames).to(BF16)
    e = linear(linear(s, p.time1_w, p.time1_b, act_out="silu"), p.time2_w, p.time2_b)
    e0 = linear(e, p.proj_w, p.proj_b, silu_in=True)
    return e, e0.view(e.shape[0], 6, -1)


def text_embed(p, context, text_len=512):
    """context [L, text_dim] bf16, padded with zero rows to text_len -> [text_len, dim] bf16."""
    ctx = torch.cat([context, context.new_zeros(text_len - context.shape[0], context.shape[1])])
    return linear(linear(ctx, p.text1_w, p.text1_b, act_out="gelu"), p.text2_w, p.text2_b)


def head(p, x, e):
    """x [T, dim] bf16, e [F, dim] bf16 (time embedding) -> [T, 64] bf16."""
    Fr = e.shape[0]
    es = p.head_mod[0].unsqueeze(0) + e.unsqueeze(1)          # [F, 2, dim] bf16
    ft = x.shape[0] // Fr
    shift = es[:, 0].repeat_interleave(ft, dim=0)
    scale = es[:, 1].repeat_interleave(ft, dim=0)
    h = F.layer_norm(x, (x.shape[-1],), None, None, EPS)
    return linear(h * (1 + scale) + shift, p.head_w, p.head_b)


def unpatchify(y, grid, c=16):
    """y [F*H'*W', 4c] -> [c, F, 2H', 2W'] ('fhwpqrc->cfphqwr', patch (1, 2, 2))."""
    Fr, hp, wp = grid
    u = y.view(Fr, hp, wp, 1, 2, 2, c)
    u = torch.einsum("fhwpqrc->cfphqwr", u)
    return u.reshape(c, Fr, hp * 2, wp * 2)


def sigma_x0(sigmas, timesteps, t: float) -> float:
    """sigma of the timestep nearest to t, in float64 (wan_wrapper.py:182-190)."""
    ts = timesteps.double()
    idx = torch.argmin((ts.unsqueeze(0) - torch.tensor([float(t)], dtype=torch.float64).unsqueeze(1)).abs(), dim=1)
    return float(sigmas.double()[idx])


def flow_to_x0(flow, xt, sigma: float):
    """x0 = xt - sigma * flow in float64, cast to bf16 (wan_wrapper.py:169-193)."""
    return (xt.double() - sigma * flow.double()).to(BF16)


def forward_head_x0(p, x, e, xt_cfhw, sigma, c=16):
    """Head + unpatchify + flow -> x0 of one chunk: x [T, dim], xt [c, F, H, W] -> x0 [F, c, H, W] bf16."""
    _, Fr, H, W = xt_cfhw.shape
    flow = unpatchify(head(p, x, e), (Fr, H // 2, W // 2), c)
    return flow_to_x0(flow, xt_cfhw, sigma).permute(1, 0, 2, 3).contiguous()


def dit_forward(p, stack_fn, latent_cfhw, t: float, sigma: float, c=16):
    """One chunk: patch embedding, time embedding, the blocks (stack_fn(x, e0) -> x), head, x0 [F, c, H, W]."""
    Fr = latent_cfhw.shape[1]
    x = patch_embed(latent_cfhw, p.patch_w, p.patch_b)
    e, e0 = time_embed(p, torch.full((Fr,), float(t), dtype=torch.float64))
    x = stack_fn(x, e0)
    return forward_head_x0(p, x, e, latent_cfhw, sigma, c)

