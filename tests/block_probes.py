"""Closed-form probes of the Wan block's wiring (causal_model.py:376-398).

Each probe picks weights and modulation so that the block's output has a
closed form built from pieces pinned elsewhere (the int8 linear, the FP8 row
codec, bf16 rounding), and so that a plausible wiring mistake changes it:

* ``residuals``: every linear weight zero, biases random.  Each linear then
  returns exactly its bf16 bias, so
      x1 = bf16(x  + bf16(o_b      * g2))     (self-attention, gate chunk 2)
      x2 = bf16(x1 + co_b)                    (cross-attention, no gate)
      x3 = bf16(x2 + bf16(fc_out_b * g5))     (FFN, gate chunk 5)
  with g_k = bf16(modulation[k] + e[:, k]) per frame.  Pins the gates and the
  order of the three residual branches (bf16 rounding is not associative).
* ``ffn_mod``: as ``residuals`` but random FFN weights, modulation[4] = 0 and
  e[:, 4] = -1, so LN2(x2) * (1 + g4) + g3 = g3 exactly and the FFN sees the
  frame's shift row: x3 = bf16(x2 + bf16(FFN(g3) * g5)).  Pins shift = chunk
  3, scale = chunk 4 and that the FFN reads the modulated norm2 output.
* ``attn_mod``: modulation[1] = 0, e[:, 1] = -1 and one e[:, 0] row for all
  frames, so LN1(x) * (1 + g1) + g0 = g0 for every token: V is one row,
  the attention over the chunk's own pages returns its FP8 dequantization
  for every query, and x1 = bf16(x + bf16(o(V) * g2)).  Pins shift = chunk
  0, scale = chunk 1 and the V projection of the modulated norm1 output.
* ``cross``: random cross-attention weights over a text context of one
  repeated row, so the cross-attention returns that row's value projection
  for every query: x2 = bf16(x1 + co(cv(text row))).  Pins the ungated
  cross-attention residual and its text value path.

``alternatives`` builds the same closed forms with a chunk or the branch order
changed; a probe is only useful if they differ from the true one.
"""

from __future__ import annotations

import dataclasses

import torch

from oracle import kv as okv
from oracle import linear as olin
from waveforcing_amd.block import random_block_params

DIM, HEADS, FFN = 256, 2, 512
FRAMES, HT, WD = 3, 8, 8
T = FRAMES * HT * WD
PAGE = HT * WD
TEXT = 16

ATTN_W = ("q_w", "k_w", "v_w", "o_w")
CROSS_W = ("cq_w", "ck_w", "cv_w", "co_w")
FFN_W = ("fc_in_w", "fc_out_w")


def bf(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16)


def _zero(p, names):
    return dataclasses.replace(p, **{n: torch.zeros_like(getattr(p, n)) for n in names})


def _per_frame(rows: torch.Tensor) -> torch.Tensor:
    """[F, dim] frame rows -> [T, dim] token rows."""
    return rows.repeat_interleave(T // FRAMES, dim=0)


def _gates(p, e):
    """g[k] = bf16(modulation[k] + e[:, k]) as [T, dim] token rows, k = 0..5."""
    es = p.modulation[0].unsqueeze(0) + e
    return [_per_frame(es[:, k]) for k in range(6)]


def _gate_add(x, y, g):
    return bf(x.float() + bf(y.float() * g.float()).float())


def _add(x, y):
    return bf(x.float() + y.float())


def _ffn(p, h):
    return olin.i8_linear(olin.i8_linear(h, p.fc_in_w, p.fc_in_b, gelu=True), p.fc_out_w, p.fc_out_b)


def build(kind: str, seed: int = 0) -> dict:
    """Inputs of a probe and its expected block output (bf16 [T, dim])."""
    p = random_block_params(DIM, FFN, seed=100 + seed)
    g = torch.Generator().manual_seed(200 + seed)
    x = bf(torch.randn((T, DIM), generator=g))
    e = bf(torch.randn((FRAMES, 6, DIM), generator=g) * 0.5)
    text = bf(torch.randn((TEXT, DIM), generator=g))
    mod = p.modulation.clone()
    if kind == "residuals":
        p = _zero(p, ATTN_W + CROSS_W + FFN_W)
    elif kind == "ffn_mod":
        p = _zero(p, ATTN_W + CROSS_W)
        mod[0, 4] = 0
        e[:, 4] = -1
    elif kind == "attn_mod":
        p = _zero(p, ("q_w", "k_w") + CROSS_W + FFN_W)
        mod[0, 1] = 0
        e[:, 1] = -1
        e[:, 0] = e[0, 0]
    elif kind == "cross":
        p = _zero(p, ATTN_W + FFN_W)
        text = text[:1].expand(TEXT, DIM).contiguous()
    else:
        raise ValueError(kind)
    p = dataclasses.replace(p, modulation=mod)
    return dict(kind=kind, params=p, x=x, e=e, text=text, expected=expected(kind, p, x, e, text))


def _attn_out(kind, p, e):
    """bf16 [T, dim] output of the self-attention branch before its gate."""
    if kind != "attn_mod":
        return _per_frame(p.o_b.unsqueeze(0).expand(FRAMES, DIM))
    g = _gates(p, e)
    a = g[0][:1]                                      # every token's modulated norm1 output
    v = olin.i8_linear(a, p.v_w, p.v_b).view(1, HEADS, DIM // HEADS)
    v_deq = okv.dequantize_rows(*okv.quantize_rows(v)).reshape(1, DIM)
    return olin.i8_linear(v_deq, p.o_w, p.o_b).expand(T, DIM)


def _cross_out(kind, p, text):
    if kind != "cross":
        return p.co_b.unsqueeze(0).expand(T, DIM)
    v = olin.i8_linear(text[:1], p.cv_w, p.cv_b)
    return olin.i8_linear(v, p.co_w, p.co_b).expand(T, DIM)


def _ffn_out(kind, p, e):
    if kind != "ffn_mod":
        return p.fc_out_b.unsqueeze(0).expand(T, DIM)
    es = p.modulation[0].unsqueeze(0) + e
    return _per_frame(_ffn(p, es[:, 3]))


def expected(kind, p, x, e, text, gate_attn=2, gate_ffn=5, order=("attn", "cross", "ffn")):
    g = _gates(p, e)
    steps = {
        "attn": lambda v: _gate_add(v, _attn_out(kind, p, e), g[gate_attn]),
        "cross": lambda v: _add(v, _cross_out(kind, p, text)),
        "ffn": lambda v: _gate_add(v, _ffn_out(kind, p, e), g[gate_ffn]),
    }
    out = x
    for s in order:
        out = steps[s](out)
    return out


def alternatives(probe: dict) -> list[torch.Tensor]:
    """Closed forms with another gate chunk or another residual order."""
    p, x, e, text, kind = probe["params"], probe["x"], probe["e"], probe["text"], probe["kind"]
    out = [expected(kind, p, x, e, text, gate_attn=k) for k in range(6) if k != 2]
    out += [expected(kind, p, x, e, text, gate_ffn=k) for k in range(6) if k != 5]
    out += [expected(kind, p, x, e, text, order=o) for o in
            (("attn", "ffn", "cross"), ("cross", "attn", "ffn"), ("ffn", "cross", "attn"))]
    return out


def pools():
    """Zeroed CPU pools of one chunk (own pages 0..FRAMES-1)."""
    return okv.new_pool(FRAMES, PAGE, HEADS, 128), okv.new_pool(FRAMES, PAGE, HEADS, 128)
