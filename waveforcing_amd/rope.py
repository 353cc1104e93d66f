"""3-D RoPE tables of the Wan DiT (host side, computed once per geometry).

The rotary frequencies follow rope_params (naive_rt/rolling_forcing/wan/
modules/model.py:29-36: angle(pos, i) = pos / theta^(2i / dim), float64) with
the head's 64 complex pairs split 22 / 21 / 21 between frame, height and
width (causal_model.py:31,549-552; the same split as _anchor_rope,
wave_rt/denoiser/exchange/common.py:51-55).  A token of grid position
(f, y, x) in a chunk starting at latent frame ``start_frame`` rotates pair i
by (start_frame + f) * w_t[i], y * w_h[i - 22] or x * w_w[i - 43]
(causal_rope_apply, causal_model.py:36-50).  Tables are produced in float64
and stored as fp32 cos/sin [T, head_dim / 2], as SGLang's
get_rotary_pos_embed is used (common.py:56-66).
"""

from __future__ import annotations

import torch

_CACHE: dict = {}
_CACHE_MAX = 64


def split_pairs(head_dim: int) -> tuple[int, int, int]:
    c = head_dim // 2
    return c - 2 * (c // 3), c // 3, c // 3


def angles(frames: int, height: int, width: int, start_frame: int = 0, head_dim: int = 128,
           theta: float = 10000.0) -> torch.Tensor:
    """float64 [frames*height*width, head_dim/2] rotation angles."""
    nt, nh, nw = split_pairs(head_dim)

    def inv(n):  # rope_params(max_len, dim=2n) frequencies
        return 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float64),
                               torch.arange(0, 2 * n, 2, dtype=torch.float64) / (2 * n))

    f = torch.arange(start_frame, start_frame + frames, dtype=torch.float64)
    y = torch.arange(height, dtype=torch.float64)
    x = torch.arange(width, dtype=torch.float64)
    at = (f[:, None] * inv(nt)[None, :])[:, None, None, :].expand(frames, height, width, nt)
    ah = (y[:, None] * inv(nh)[None, :])[None, :, None, :].expand(frames, height, width, nh)
    aw = (x[:, None] * inv(nw)[None, :])[None, None, :, :].expand(frames, height, width, nw)
    return torch.cat([at, ah, aw], dim=-1).reshape(frames * height * width, nt + nh + nw)


def cos_sin(frames: int, height: int, width: int, start_frame: int = 0, head_dim: int = 128,
            device="cuda") -> tuple[torch.Tensor, torch.Tensor]:
    """Cached fp32 (cos, sin) [T, head_dim/2] on ``device`` (cache key as _anchor_rope's)."""
    key = (frames, height, width, start_frame, head_dim, str(device))
    hit = _CACHE.get(key)
    if hit is None:
        # the anchor's start frame moves every step of a long stream: keep the cache bounded
        if len(_CACHE) >= _CACHE_MAX:
            _CACHE.pop(next(iter(_CACHE)))
        a = angles(frames, height, width, start_frame, head_dim)
        hit = (torch.cos(a).float().contiguous().to(device), torch.sin(a).float().contiguous().to(device))
        _CACHE[key] = hit
    return hit
