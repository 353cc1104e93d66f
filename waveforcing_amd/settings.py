"""Environment-controlled constants of the quantized block path.

Mirrors the FP8 part of wave_rt/denoiser/settings.py:20-24 and the flag parser
of wave_rt/runtime/env.py:8-13 (same flag names, same parsing rules).
"""

from __future__ import annotations

import os

import torch

_FALSE_VALUES = {"", "0", "false"}


def env_flag(name: str, *, default: bool = False) -> bool:
    """Boolean env flag: unset, "", "0" and "false" are false (wave_rt/runtime/env.py:10-13)."""
    fallback = "1" if default else ""
    return os.environ.get(name, fallback) not in _FALSE_VALUES


FP8_KV = env_flag("WAVE_FP8_KV")
FP8_KV_ONESIDED = env_flag("WAVE_FP8KV_ONESIDED")
FP8_E4M3_MAX = 448.0
FP8_DTYPE = torch.float8_e4m3fn
GENERATION_SLOTS = int(os.environ.get("WAVE_OS_GT", "2"))

# One latent frame of the 480x832 Wan2.1 geometry is 1560 tokens
# (naive_rt/rolling_forcing/wan/modules/causal_model.py:75); a chunk is three
# frames (causal_model.py:77).  A KV page holds one frame.
FRAME_TOKENS = 1560
FRAMES_PER_CHUNK = 3
CHUNK_TOKENS = FRAME_TOKENS * FRAMES_PER_CHUNK
PAGE_TOKENS = FRAME_TOKENS
HEAD_DIM = 128
