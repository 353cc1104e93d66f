"""Pins the DiT oracle (oracle/dit.py) on the CPU.

- the patch embedding equals torch's F.conv3d with kernel = stride = (1, 2, 2)
  followed by flatten(2).transpose(1, 2) (the reference's own call,
  causal_model.py:517-518,826-830), to fp32 summation order;
- unpatchify inverts the patch gather read in the head's (q, r, c) order, so
  the 'fhwpqrc->cfphqwr' layout is pinned independently of the gather;
- sinusoidal_embedding_1d against its closed form cos / sin(t * 10000^(-i/128));
- zero linear weights leave exactly the bias path (time embedding, projection,
  head), and a one-hot head weight reads back a chosen input column;
- flow -> x0: sigma = 0 returns xt, exact cases of xt - sigma * flow, and the
  float64 -> bf16 conversion goes through float32 as torch's does;
- sigma at the warped DMD timesteps is the closed form 5s / (1 + 4s) of the
  shifted schedule (1, 15/16, 5/6, 5/8), and the product's lookup equals it;
- the activations of the time and text embeddings (causal_model.py:519-525,
  840-855): with one-hot weights (tests/embed_probes.py) the time embedding
  is bf16(silu(.)) of chosen sinusoid columns and the projection
  bf16(silu(.)) of chosen e columns, the text embedding bf16(gelu_tanh(.)) of
  chosen context columns plus the second bias (the bias alone on the padding
  rows), each within one bf16 ulp of its float64 definition; a dropped SiLU,
  a dropped GELU or a SiLU in the GELU's place moves most elements further.
"""

import dataclasses
import math

import pytest

import torch
import torch.nn.functional as F

import embed_probes as ep
from oracle import dit as od
from oracle import schedule as osch
from waveforcing_amd.dit import random_dit_params
from waveforcing_amd.schedule import FlowMatchSchedule

BF16 = torch.bfloat16


def _latent(C=16, Fr=3, H=8, W=12, seed=0):
    return torch.randn((C, Fr, H, W), generator=torch.Generator().manual_seed(seed)).to(BF16)


def _ulp(x):
    return torch.pow(2.0, torch.floor(torch.log2(x.abs().clamp(min=2.0 ** -100))) - 7)


def test_patch_embed_equals_conv3d():
    p = random_dit_params(96, seed=1)
    lat = _latent()
    got = od.patch_embed(lat, p.patch_w, p.patch_b).float()
    conv = F.conv3d(lat.float()[None], p.patch_w.float(), p.patch_b.float(), stride=(1, 2, 2))
    want = conv.flatten(2).transpose(1, 2)[0]
    assert got.shape == want.shape == (3 * 4 * 6, 96)
    # one bf16 rounding of the same fp32 sum (order of the 64 products may differ)
    assert ((got - want).abs() <= _ulp(want) + 1e-6).all()
    assert (got == want.to(BF16).float()).double().mean() > 0.99


def test_unpatchify_inverts_patch_gather_in_head_order():
    lat = _latent(C=16, Fr=2, H=6, W=10, seed=2)
    C, Fr, H, W = lat.shape
    pat = od.patchify(lat).view(-1, C, 2, 2)                   # [T, c, kh, kw]
    head_order = pat.permute(0, 2, 3, 1).reshape(-1, 4 * C)    # [T, (q, r, c)]
    assert torch.equal(od.unpatchify(head_order, (Fr, H // 2, W // 2), C), lat)
    # and the gather itself reads the 2 x 2 patch of each channel
    assert torch.equal(pat[0, 5], lat[5, 0, 0:2, 0:2])
    assert torch.equal(pat[(1 * 3 + 2) * 5 + 4, 7], lat[7, 1, 4:6, 8:10])


def test_sinusoidal_embedding_closed_form():
    t = torch.tensor([0.0, 1000.0, 937.5], dtype=torch.float64)
    s = od.sinusoidal_embedding_1d(256, t)
    assert torch.equal(s[0], torch.cat([torch.ones(128), torch.zeros(128)]).double())
    for i in (0, 1, 64, 127):
        w = 10000.0 ** (-i / 128)
        assert math.isclose(float(s[1, i]), math.cos(1000.0 * w), rel_tol=0, abs_tol=1e-12)
        assert math.isclose(float(s[2, 128 + i]), math.sin(937.5 * w), rel_tol=0, abs_tol=1e-12)


def test_zero_weights_leave_bias_paths():
    p = random_dit_params(64, seed=3)
    z = {n: torch.zeros_like(getattr(p, n)) for n in ("time1_w", "time2_w", "proj_w", "head_w")}
    p = dataclasses.replace(p, **z)
    e, e0 = od.time_embed(p, torch.tensor([937.5, 937.5, 937.5], dtype=torch.float64))
    assert torch.equal(e, p.time2_b.expand(3, -1))
    assert torch.equal(e0, p.proj_b.view(6, 64).expand(3, 6, 64))
    x = torch.randn((3 * 16, 64), generator=torch.Generator().manual_seed(4)).to(BF16)
    assert torch.equal(od.head(p, x, e), p.head_b.expand(48, -1))


def test_head_reads_the_modulated_layer_norm():
    p = random_dit_params(64, seed=5)
    # one-hot head weight: output column o reads input column 10, no bias
    hw = torch.zeros_like(p.head_w)
    hw[:, 10] = 1
    p = dataclasses.replace(p, head_w=hw, head_b=torch.zeros_like(p.head_b))
    x = torch.randn((2 * 8, 64), generator=torch.Generator().manual_seed(6)).to(BF16)
    e = torch.randn((2, 64), generator=torch.Generator().manual_seed(7)).to(BF16)
    es = p.head_mod[0].unsqueeze(0) + e.unsqueeze(1)
    ln = F.layer_norm(x, (64,), None, None, 1e-6)
    frame = torch.arange(16) // 8
    want = (ln[:, 10] * (1 + es[frame, 1, 10]) + es[frame, 0, 10]).float()
    got = od.head(p, x, e)
    assert torch.equal(got.float(), want.unsqueeze(1).expand(16, 64).to(BF16).float())


def test_flow_to_x0_exact_cases_and_float32_route():
    g = torch.Generator().manual_seed(8)
    xt = torch.randn((16, 3, 4, 4), generator=g).to(BF16)
    flow = torch.randn((16, 3, 4, 4), generator=g).to(BF16)
    assert torch.equal(od.flow_to_x0(flow, xt, 0.0), xt)
    # sigma = 1/2 on values with few significant bits: exact in float64 and in bf16
    a = torch.tensor([1.5, -2.0, 0.25], dtype=BF16)
    b = torch.tensor([1.0, 4.0, -0.5], dtype=BF16)
    assert torch.equal(od.flow_to_x0(b, a, 0.5), torch.tensor([1.0, -4.0, 0.5], dtype=BF16))
    # a float64 result just above a bf16 midpoint rounds down through float32, as torch converts
    d = 1 + 2 ** -8 + 2 ** -30
    one = torch.tensor([d], dtype=torch.float64)
    assert float(one.to(BF16)) == 1.0 and float(one.float().to(BF16)) == 1.0


def test_sigma_at_warped_steps_closed_form_and_product_lookup():
    sig, ts = osch.flow_sigmas()
    steps = osch.warp_steps(ts, (1000, 750, 500, 250))
    sched = FlowMatchSchedule()
    for t, want in zip(steps.tolist(), (1.0, 15 / 16, 5 / 6, 5 / 8)):
        s = od.sigma_x0(sig, ts, t)
        assert abs(s - want) < 1e-6
        assert sched.sigma_x0(t) == s
    # between two table entries the nearer one wins (the first on a tie)
    assert od.sigma_x0(sig, ts, float(ts[10]) + 1e-3) == float(sig[10].double())


@pytest.mark.parametrize("t", [1000.0, 937.5, 625.0, 3.0])
def test_time_embedding_activations_closed_form(t):
    p, picks = ep.time_probe(random_dit_params(64, seed=9))
    e, e0 = od.time_embed(p, torch.full((3,), t, dtype=torch.float64))
    want_e, want_e0 = ep.time_closed_form(t, 3, picks)
    assert ep.within_one_ulp(e, want_e) and ep.within_one_ulp(e0, want_e0)
    for name, (ae, ae0) in ep.time_alternatives(t, 3, picks).items():
        far = max(ep.far_fraction(ae, want_e), ep.far_fraction(ae0, want_e0))
        assert far > 0.3, f"{name}: only {far:.2f} of the elements move"


def test_text_embedding_activation_and_padding_closed_form():
    p, ctx, picks = ep.text_probe(random_dit_params(64, seed=10))
    got = od.text_embed(p, ctx)
    want = ep.text_closed_form(ctx, p.text2_b, picks)
    assert got.shape == (512, 64)
    assert ep.within_one_ulp(got, want)
    # the rows that pad the context to 512 read back the second bias exactly
    assert torch.equal(got[ctx.shape[0]:], p.text2_b.expand(512 - ctx.shape[0], 64))
    for name, alt in ep.text_alternatives(ctx, p.text2_b, picks).items():
        far = ep.far_fraction(alt[:ctx.shape[0]], want[:ctx.shape[0]])
        assert far > 0.3, f"{name}: only {far:.2f} of the context rows' elements move"
