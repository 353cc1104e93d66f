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

The q/k RMSNorm wiring (causal_model.py:112-116, model.py:171-178) has probes
of its own, built so that every normalized vector has a closed form: a linear
whose output is +-2 in every column (zero weight, bias 2 * sign) normalizes
to exactly +-1 in bf16 (2 * rsqrt(4 + 1e-6) rounds to 1), so RMSNorm(.) * w
is sign * w element by element.

* ``self_qk``: x = 0 (so LN1(x) = 0 and the modulated norm1 output is the
  frame's shift row g0), q and k linears as above, norm weights ~2.5 that
  differ between norm_q and norm_k: every token's pre-RoPE query is
  sq * norm_q and key sk * norm_k; V is the value projection of the frame's
  g0 row, so the attention output weighs three distinct value rows by scores
  that depend on both norm weights.
* ``cross_q``: cross-attention query linear zero with bias 2 * sign, so
  every token's query is sq * cnorm_q; the text rows are a_j * tau_j (a_j a
  power of two, tau_j a sign vector) and the text key/value linears are
  scaled identities, so text_kv returns K_j = tau_j * cnorm_k and
  V_j = a_j * c_v * tau_j exactly (``text_kv_closed_form``).  Exchanging
  cnorm_q and cnorm_k together leaves every score sum_d q_d k_d unchanged
  (each term holds the product cnorm_q[d] * cnorm_k[d]), so that exchange
  is invisible to any input, in the reference as here, and is not a probe
  target; either weight taken for both, or a norm dropped, is.

``qk_alternatives`` gives the closed forms of the plausible mistakes: a norm
weight taken from the other norm of the pair, a norm dropped, or a query and
key normalized with one weight.
"""

from __future__ import annotations

import dataclasses

import torch

from oracle import attention as oat
from oracle import block as ob
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
    elif kind == "self_qk":
        x = torch.zeros_like(x)
        p = _zero(p, ("q_w", "k_w") + CROSS_W + FFN_W)
        p = dataclasses.replace(p, q_b=bf(2 * _signs(DIM, g)), k_b=bf(2 * _signs(DIM, g)),
                                norm_q=_norm_weight(g), norm_k=_norm_weight(g),
                                v_w=bf(p.v_w.float() * 10), o_w=bf(p.o_w.float() * 10))
    elif kind == "cross_q":
        x = torch.zeros_like(x)
        p = _zero(p, ATTN_W + FFN_W + ("cq_w",))
        text = _sign_text(g)
        p = dataclasses.replace(p, cq_b=bf(2 * _signs(DIM, g)), cnorm_q=_norm_weight(g), cnorm_k=_norm_weight(g),
                                ck_w=bf(TEXT_CK * torch.eye(DIM)), ck_b=torch.zeros_like(p.ck_b),
                                cv_w=bf(TEXT_CV * torch.eye(DIM)), cv_b=torch.zeros_like(p.cv_b),
                                co_w=bf(p.co_w.float() * 10))
    else:
        raise ValueError(kind)
    p = dataclasses.replace(p, modulation=mod)
    return dict(kind=kind, params=p, x=x, e=e, text=text, expected=expected(kind, p, x, e, text))


# ---------------------------------------------------------------- q/k RMSNorm wiring
TEXT_CK, TEXT_CV = 0.5, 0.25          # scaled-identity text key / value linears (powers of two)
TEXT_AMP = (0.5, 1.0, 2.0, 4.0)       # text row amplitudes a_j (powers of two)


def _signs(n, g):
    return torch.where(torch.rand(n, generator=g) < 0.5, -1.0, 1.0)


def _norm_weight(g):
    """A norm weight ~2.5 +- 0.6 (bf16): scores of several units, so that a weight taken from the wrong norm
    moves the softmax by far more than rounding does (each mistake changes the block output by >= 10 %)."""
    return bf(2.5 + 0.6 * torch.randn(DIM, generator=g))


def _sign_text(g):
    """Text rows a_j * tau_j with a_j from TEXT_AMP and tau_j a random sign vector: [TEXT, DIM] bf16."""
    amp = torch.tensor([TEXT_AMP[j % len(TEXT_AMP)] for j in range(TEXT)]).unsqueeze(1)
    return bf(amp * torch.stack([_signs(DIM, g) for _ in range(TEXT)]))


def _sign_of(t):
    return torch.sign(t.float())


def text_kv_closed_form(p, text, k_weight=None, k_norm=True):
    """K, V of the sign-vector text through scaled-identity linears: K_j = tau_j * cnorm_k and
    V_j = a_j * TEXT_CV * tau_j, [TEXT, HEADS, 128] bf16.  ``k_weight`` / ``k_norm=False`` give the closed
    forms of a text key normalized with another weight or not normalized at all."""
    w = p.cnorm_k if k_weight is None else k_weight
    tau = _sign_of(text)
    if k_norm:
        k = bf(tau * w.float())
    else:
        k = bf(text.float() * TEXT_CK)
    v = bf(text.float() * TEXT_CV)
    return k.view(TEXT, HEADS, DIM // HEADS), v.view(TEXT, HEADS, DIM // HEADS)


def _query(bias, weight, norm=True):
    """The closed-form query of a zero-weight linear with bias 2 * sign: sign * weight, or the raw bias."""
    return bf(_sign_of(bias) * weight.float()) if norm else bias


def _self_attn_qk(p, e, q_weight=None, k_weight=None, q_norm=True, k_norm=True):
    """bf16 [T, DIM] self-attention branch output (before its gate) of the ``self_qk`` probe."""
    hd = DIM // HEADS
    q = _query(p.q_b, p.norm_q if q_weight is None else q_weight, q_norm)
    k = _query(p.k_b, p.norm_k if k_weight is None else k_weight, k_norm)
    ang = ob.rope_angles(FRAMES, HT, WD, 0, hd)
    q_r = ob.rope_apply(q.expand(T, DIM).reshape(T, HEADS, hd), ang)
    k_r = ob.rope_apply(k.expand(T, DIM).reshape(T, HEADS, hd), ang)
    g0 = _gates(p, e)[0]                                   # LN1(0) * (1 + g1) + g0 = g0
    v = olin.i8_linear(g0, p.v_w, p.v_b).view(T, HEADS, hd)
    k_deq = okv.dequantize_rows(*okv.quantize_rows(k_r))
    v_deq = okv.dequantize_rows(*okv.quantize_rows(v))
    y = oat.sdpa(q_r, k_deq, v_deq).to(torch.bfloat16).reshape(T, DIM)
    return olin.i8_linear(y, p.o_w, p.o_b)


def _cross_attn_q(p, text, q_weight=None, q_norm=True, k_weight=None, k_norm=True):
    """bf16 [T, DIM] cross-attention branch output of the ``cross_q`` probe."""
    q = _query(p.cq_b, p.cnorm_q if q_weight is None else q_weight, q_norm).view(1, HEADS, DIM // HEADS)
    k, v = text_kv_closed_form(p, text, k_weight, k_norm)
    y = oat.sdpa(q, k, v).to(torch.bfloat16).reshape(1, DIM)
    return olin.i8_linear(y, p.co_w, p.co_b).expand(T, DIM)


def qk_alternatives(probe: dict) -> dict:
    """name -> closed form of the probe's block output with one q/k norm wired wrongly."""
    p, x, e, text, kind = probe["params"], probe["x"], probe["e"], probe["text"], probe["kind"]
    if kind == "self_qk":
        variants = {
            "k normalized with norm_q": dict(k_weight=p.norm_q),
            "q normalized with norm_k": dict(q_weight=p.norm_k),
            "norm_q and norm_k swapped": dict(q_weight=p.norm_k, k_weight=p.norm_q),
            "no q RMSNorm": dict(q_norm=False),
            "no k RMSNorm": dict(k_norm=False),
        }
        return {n: expected(kind, p, x, e, text, attn_fn=lambda kw=kw: _self_attn_qk(p, e, **kw))
                for n, kw in variants.items()}
    if kind == "cross_q":
        variants = {
            "text K normalized with cnorm_q": dict(k_weight=p.cnorm_q),
            "query normalized with cnorm_k": dict(q_weight=p.cnorm_k),
            "no cross q RMSNorm": dict(q_norm=False),
            "no text K RMSNorm": dict(k_norm=False),
        }
        return {n: expected(kind, p, x, e, text, cross_fn=lambda kw=kw: _cross_attn_q(p, text, **kw))
                for n, kw in variants.items()}
    raise ValueError(kind)


def _attn_out(kind, p, e):
    """bf16 [T, dim] output of the self-attention branch before its gate."""
    if kind == "self_qk":
        return _self_attn_qk(p, e)
    if kind != "attn_mod":
        return _per_frame(p.o_b.unsqueeze(0).expand(FRAMES, DIM))
    g = _gates(p, e)
    a = g[0][:1]                                      # every token's modulated norm1 output
    v = olin.i8_linear(a, p.v_w, p.v_b).view(1, HEADS, DIM // HEADS)
    v_deq = okv.dequantize_rows(*okv.quantize_rows(v)).reshape(1, DIM)
    return olin.i8_linear(v_deq, p.o_w, p.o_b).expand(T, DIM)


def _cross_out(kind, p, text):
    if kind == "cross_q":
        return _cross_attn_q(p, text)
    if kind != "cross":
        return p.co_b.unsqueeze(0).expand(T, DIM)
    v = olin.i8_linear(text[:1], p.cv_w, p.cv_b)
    return olin.i8_linear(v, p.co_w, p.co_b).expand(T, DIM)


def _ffn_out(kind, p, e):
    if kind != "ffn_mod":
        return p.fc_out_b.unsqueeze(0).expand(T, DIM)
    es = p.modulation[0].unsqueeze(0) + e
    return _per_frame(_ffn(p, es[:, 3]))


def expected(kind, p, x, e, text, gate_attn=2, gate_ffn=5, order=("attn", "cross", "ffn"), attn_fn=None,
             cross_fn=None):
    g = _gates(p, e)
    attn = attn_fn if attn_fn is not None else (lambda: _attn_out(kind, p, e))
    cross = cross_fn if cross_fn is not None else (lambda: _cross_out(kind, p, text))
    steps = {
        "attn": lambda v: _gate_add(v, attn(), g[gate_attn]),
        "cross": lambda v: _add(v, cross()),
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
