"""Pins the block oracle (oracle/block.py) on the CPU.

- zero linear weights and biases leave x unchanged (every branch is a
  residual; no stray term);
- RoPE: position (0, 0, 0) of a chunk starting at frame 0 is the identity,
  rotations preserve each pair's norm, and the angle table equals the host
  table generator's (waveforcing_amd.rope, written separately);
- the norms match torch's layer_norm / the closed-form RMS definition in
  float64;
- the table form of RoPE (fp32 cos/sin, fp32 arithmetic, one bf16 rounding)
  agrees with the float64 complex rotation to one bf16 ulp and exactly in
  all but a few near-tie elements, is exact for the rotations by 0, 90 and
  180 degrees, and equals a scalar numpy-float32 evaluation element by
  element;
- the wiring of causal_model.py:376-398 (which modulation chunk is which
  shift, scale and gate, which norm feeds which branch, the order of the
  three residuals) equals the closed forms of tests/block_probes.py exactly;
  every swap of two modulation chunks and every other residual order changes
  at least one probe's output;
- the q/k RMSNorm wiring (causal_model.py:112-116, model.py:171-178): the
  self-attention and cross-attention probes of tests/block_probes.py give
  the oracle block exactly their closed forms (queries and keys sign * norm
  weight, through the pinned RoPE, FP8 row codec, int8 linear and SDPA), the
  oracle's text K/V equal tau_j * cnorm_k and a_j * c_v * tau_j bit for bit,
  and each plausible mistake (a norm weight from the other norm, a norm
  dropped) moves the closed form by more than 5 % relative L2.
"""

import dataclasses
import itertools

import pytest

import numpy as np
import torch

import block_probes as bp
from oracle import block as ob
from oracle import kv as okv
from waveforcing_amd import rope
from waveforcing_amd.block import random_block_params


def test_zero_weights_identity():
    dim, heads, ffn = 256, 2, 512
    p = random_block_params(dim, ffn, seed=1)
    zero = {f.name: torch.zeros_like(getattr(p, f.name)) for f in dataclasses.fields(p)
            if f.name.endswith(("_w", "_b")) and not f.name.startswith("norm3")}
    p = dataclasses.replace(p, **zero)
    frames, h, w = 3, 8, 8
    T = frames * h * w
    g = torch.Generator().manual_seed(2)
    x = torch.randn((T, dim), generator=g).to(torch.bfloat16)
    e = (torch.randn((frames, 6, dim), generator=g) * 0.1).to(torch.bfloat16)
    pk = okv.new_pool(3, 64, heads, 128)
    pv = okv.new_pool(3, 64, heads, 128)
    tk = torch.zeros((16, heads, 128), dtype=torch.bfloat16)
    out = ob.block_forward(p, x, e, (frames, h, w), 0, pk, pv, [0, 1, 2], [0, 1, 2], T, 64, tk, tk, heads)
    assert torch.equal(out, x)


def test_rope_identity_norm_and_table():
    ang = ob.rope_angles(3, 4, 5, 0)
    assert torch.equal(ang[0], torch.zeros(64, dtype=torch.float64))
    assert torch.allclose(ang, rope.angles(3, 4, 5, 0), rtol=0, atol=0)
    assert torch.allclose(ob.rope_angles(3, 4, 5, 7), rope.angles(3, 4, 5, 7), rtol=0, atol=0)
    g = torch.Generator().manual_seed(3)
    x = torch.randn((60, 2, 128), generator=g).to(torch.bfloat16)
    y = ob.rope_apply(x, ob.rope_angles(3, 4, 5, 2))
    assert torch.equal(ob.rope_apply(x[:1], torch.zeros((1, 64), dtype=torch.float64)), x[:1])
    nx = x.double().reshape(60, 2, 64, 2).norm(dim=-1)
    ny = y.double().reshape(60, 2, 64, 2).norm(dim=-1)
    assert torch.allclose(nx, ny, rtol=2 ** -7, atol=1e-6)


def test_norms_match_definitions():
    g = torch.Generator().manual_seed(4)
    x = torch.randn((32, 384), generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(384, generator=g)).to(torch.bfloat16)
    xd = x.double()
    ln = (xd - xd.mean(-1, keepdim=True)) / torch.sqrt(xd.var(-1, unbiased=False, keepdim=True) + 1e-6)
    assert torch.allclose(ob.layer_norm(x).double(), ln, rtol=2 ** -7, atol=1e-2)
    rms = xd / torch.sqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert torch.allclose(ob.rms_norm(x, w).double(), rms, rtol=2 ** -6, atol=1e-2)


def _bf16_ulp(x):
    e = torch.floor(torch.log2(x.abs().clamp(min=2.0 ** -126)))
    return torch.pow(2.0, e - 7)


def test_rope_table_form_matches_float64_rotation():
    g = torch.Generator().manual_seed(5)
    ang = ob.rope_angles(3, 6, 7, 11)
    T = ang.shape[0]
    x = torch.randn((T, 3, 128), generator=g).to(torch.bfloat16)
    cos, sin = torch.cos(ang).float(), torch.sin(ang).float()
    got = ob.rope_apply_table(x, cos, sin).double()
    want = ob.rope_apply(x, ang).double()
    diff = (got - want).abs()
    assert (diff <= _bf16_ulp(want) + 1e-30).all()
    assert (diff > 0).double().mean() < 0.02
    # a half-split (neox) pairing or a flipped sine sign is far off
    assert (ob.rope_apply_table(x, cos, -sin).double() - want).abs().max() > 0.5


def test_rope_table_form_special_rotations():
    g = torch.Generator().manual_seed(6)
    x = torch.randn((5, 2, 128), generator=g).to(torch.bfloat16)
    one, zero = torch.ones((5, 64)), torch.zeros((5, 64))
    assert torch.equal(ob.rope_apply_table(x, one, zero), x)
    assert torch.equal(ob.rope_apply_table(x, -one, zero), -x)
    r90 = ob.rope_apply_table(x, zero, one).reshape(5, 2, 64, 2)
    xp = x.reshape(5, 2, 64, 2)
    assert torch.equal(r90[..., 0], -xp[..., 1]) and torch.equal(r90[..., 1], xp[..., 0])


def test_rope_table_form_equals_scalar_float32():
    g = torch.Generator().manual_seed(7)
    x = torch.randn((4, 1, 128), generator=g).to(torch.bfloat16)
    ang = torch.rand((4, 64), generator=g, dtype=torch.float64) * 100
    cos, sin = torch.cos(ang).float(), torch.sin(ang).float()
    got = ob.rope_apply_table(x, cos, sin).float().numpy()
    xf = x.float().numpy()
    c, s = cos.numpy(), sin.numpy()

    def bf16(v):  # round-to-nearest-even of a float32 to bf16, as float32
        u = np.array([v], dtype=np.float32).view(np.uint32)[0]
        u = (int(u) + 0x7FFF + ((int(u) >> 16) & 1)) & 0xFFFF0000
        return np.array([u], dtype=np.uint32).view(np.float32)[0]

    for t in range(4):
        for i in range(64):
            a, b = np.float32(xf[t, 0, 2 * i]), np.float32(xf[t, 0, 2 * i + 1])
            ci, si = np.float32(c[t, i]), np.float32(s[t, i])
            assert got[t, 0, 2 * i] == bf16(np.float32(a * ci) - np.float32(b * si))
            assert got[t, 0, 2 * i + 1] == bf16(np.float32(a * si) + np.float32(b * ci))


PROBES = ("residuals", "ffn_mod", "attn_mod", "cross", "self_qk", "cross_q")


def _run_probe(params, pr, e=None):
    pk, pv = bp.pools()
    tk, tv = ob.text_kv(params, pr["text"], bp.HEADS)
    return ob.block_forward(params, pr["x"], pr["e"] if e is None else e, (bp.FRAMES, bp.HT, bp.WD), 0, pk, pv,
                            [0, 1, 2], [0, 1, 2], bp.T, bp.PAGE, tk, tv, bp.HEADS)


@pytest.mark.parametrize("kind", PROBES)
def test_block_wiring_equals_closed_form(kind):
    pr = bp.build(kind)
    assert torch.equal(_run_probe(pr["params"], pr), pr["expected"])
    if kind in ("self_qk", "cross_q"):
        return  # these probe the q/k norms (test_qk_norm_mistakes_move_the_closed_form)
    # another gate chunk or another residual order is visible in this probe
    for alt in bp.alternatives(pr):
        assert not torch.equal(alt, pr["expected"])


def test_every_swap_of_two_modulation_chunks_is_caught():
    """Chunks i and j of the modulation and of e exchanged before the call is what an oracle reading chunk j
    where it should read i (and i for j) computes; some probe must see every such swap."""
    caught = set()
    for kind in PROBES:
        pr = bp.build(kind)
        for i, j in itertools.combinations(range(6), 2):
            perm = list(range(6))
            perm[i], perm[j] = j, i
            p = dataclasses.replace(pr["params"], modulation=pr["params"].modulation[:, perm])
            if not torch.equal(_run_probe(p, pr, e=pr["e"][:, perm]), pr["expected"]):
                caught.add((i, j))
    assert caught == set(itertools.combinations(range(6), 2))


@pytest.mark.parametrize("kind", ["self_qk", "cross_q"])
def test_qk_norm_mistakes_move_the_closed_form(kind):
    pr = bp.build(kind)
    want = pr["expected"].double()
    alts = bp.qk_alternatives(pr)
    assert len(alts) >= 4
    for name, alt in alts.items():
        rel = ((alt.double() - want).norm() / want.norm()).item()
        assert rel > 5e-2, f"{kind}: '{name}' is within {rel:.2e} of the true wiring"


def test_text_kv_equals_closed_form():
    pr = bp.build("cross_q")
    p, text = pr["params"], pr["text"]
    k, v = ob.text_kv(p, text, bp.HEADS)
    ck, cv = bp.text_kv_closed_form(p, text)
    assert torch.equal(k, ck) and torch.equal(v, cv)
    # the text K normalized with the query's weight, or not normalized, is another tensor
    assert not torch.equal(k, bp.text_kv_closed_form(p, text, k_weight=p.cnorm_q)[0])
    assert not torch.equal(k, bp.text_kv_closed_form(p, text, k_norm=False)[0])
