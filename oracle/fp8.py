"""e4m3fn codec oracle.

``encode`` is torch's ``.to(torch.float8_e4m3fn)``, the cast the reference
uses at wave_rt/runtime/fp8.py:35,48, wave_rt/denoiser/exchange/common.py:150
and onesided.py:152.  ``encode_bits`` is an independent numpy statement of the
OCP e4m3fn round-to-nearest-even rule (1-4-3 format, bias 7, max 448, single
NaN pattern S.1111.111, overflow to NaN), used to pin the torch cast over
every bf16 input; ``decode_closed_form`` states the decode from the format
definition.
"""

from __future__ import annotations

import numpy as np
import torch

E4M3_MAX = 448.0


def encode(x: torch.Tensor) -> torch.Tensor:
    """torch's cast: fp32/bf16 tensor -> uint8 e4m3fn codes."""
    return x.to(torch.float8_e4m3fn).view(torch.uint8)


def decode(codes: torch.Tensor) -> torch.Tensor:
    """uint8 e4m3fn codes -> fp32 via torch."""
    return codes.view(torch.float8_e4m3fn).to(torch.float32)


def encode_bits(x: np.ndarray) -> np.ndarray:
    """Independent e4m3fn RNE encoder on float32 bit patterns.

    Enumerates the finite e4m3fn magnitudes (closed form), then for each
    input picks the nearest one, breaking exact ties toward the even code;
    magnitudes above 464 (the midpoint to the non-existent 480) and NaN map
    to the NaN code.  Quadratic in the table size only (256 entries).
    """
    x = np.asarray(x, dtype=np.float32)
    finite = np.isfinite(x)
    x_safe = np.where(finite, x, np.float32(0.0))
    mags = decode_closed_form(np.arange(0, 0x7F, dtype=np.uint8))  # codes 0x00..0x7e
    ax = np.abs(x_safe.astype(np.float64))
    sign = (np.signbit(x)).astype(np.uint8) << 7
    idx = np.searchsorted(mags, ax, side="left")  # first mag >= ax
    idx = np.clip(idx, 0, len(mags) - 1)
    lo = np.clip(idx - 1, 0, len(mags) - 1)
    d_hi = mags[idx] - ax
    d_lo = ax - mags[lo]
    pick_lo = (d_lo < d_hi) | ((d_lo == d_hi) & (lo % 2 == 0) & (lo != idx))
    code = np.where(pick_lo, lo, idx).astype(np.uint8)
    code = np.where(ax <= mags[0], 0, code).astype(np.uint8)
    overflow = (ax > 464.0) | ~finite
    code = np.where(overflow, 0x7F, code).astype(np.uint8)
    return code | sign


def decode_closed_form(codes: np.ndarray) -> np.ndarray:
    """(-1)^s * 2^(e-7) * (1 + m/8) for e > 0, (-1)^s * 2^-6 * m/8 for e == 0, NaN for S.1111.111."""
    c = np.asarray(codes, dtype=np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = s * val
    return np.where((c & 0x7F) == 0x7F, np.nan, val)


def all_bf16_as_f32() -> torch.Tensor:
    """Every bf16 bit pattern, widened to fp32 (65536 values, NaNs included)."""
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16)
    return bits.view(torch.bfloat16).float()


def boundary_f32() -> torch.Tensor:
    """fp32 values at and +-4 ulps around every e4m3fn rounding boundary.

    Boundaries are the midpoints between consecutive finite magnitudes, plus
    464 (overflow edge); both signs.
    """
    mags = decode_closed_form(np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64)
    mids = (mags[1:] + mags[:-1]) / 2.0
    pts = np.concatenate([mids, mags, [464.0, 448.0]]).astype(np.float32)
    bits = pts.view(np.int32)[:, None] + np.arange(-4, 5, dtype=np.int32)[None, :]
    vals = bits.reshape(-1).view(np.float32)
    vals = vals[np.isfinite(vals) & (vals >= 0)]
    return torch.from_numpy(np.concatenate([vals, -vals]))
