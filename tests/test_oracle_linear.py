"""Pins the W8A8 linear oracle (oracle/linear.py) without the GPU.

int8 scheme: torch._int_mm equals an int64 numpy matmul; exact halfway
quotients round to even; the row max maps to +-127; the dequantized error
is at most half a step; the epilogue matches float64 within fp32 rounding;
GELU(tanh) matches its closed form.  FP8 scheme: codes and scales follow
the reference's arithmetic (a bf16 activation scale, a bf16 quotient), and
_scaled_mm equals a float64 product of the decoded codes and scales.
"""

import numpy as np
import torch

from oracle import fp8 as ofp8
from oracle import linear as olin
from waveforcing_amd import inputs


def test_int_mm_is_exact():
    g = torch.Generator().manual_seed(0)
    a = torch.randint(-127, 128, (67, 96), generator=g, dtype=torch.int8)
    b = torch.randint(-127, 128, (40, 96), generator=g, dtype=torch.int8)
    a[0] = 127
    b[0] = -127
    got = torch._int_mm(a, b.t()).numpy().astype(np.int64)
    want = a.numpy().astype(np.int64) @ b.numpy().astype(np.int64).T
    assert np.array_equal(got, want)


def test_quant_rows_ties_round_to_even_and_max_is_127():
    # rows with amax = 127 * 2^e have s = 2^e exactly; (k + 1/2) * 2^e are ties
    e = torch.tensor([-3.0, 0.0, 2.0])
    s = torch.pow(2.0, e)
    k = torch.arange(-20, 20, dtype=torch.float32)
    rows = torch.cat([torch.full((3, 1), 127.0), (k[None, :] + 0.5).expand(3, -1)], 1) * s[:, None]
    q, sx = olin.i8_quant_rows(rows)
    assert torch.equal(sx, s)
    want = torch.tensor([float(v + 0.5) for v in k.tolist()])
    want = torch.where(torch.remainder(torch.floor(want), 2) == 0, torch.floor(want), torch.ceil(want))
    assert torch.equal(q[:, 1:].float(), want.expand(3, -1))
    assert bool((q[:, 0] == 127).all())


def test_quant_rows_error_bound_and_extremes():
    x = inputs.outlier_activations(64, 512, seed=4)
    q, s = olin.i8_quant_rows(x)
    deq = q.double() * s.double()[:, None]
    assert bool(((deq - x.double()).abs() <= s.double()[:, None] * 0.5 * (1 + 1e-6)).all())
    assert bool((q.abs().amax(-1) == 127).all())
    z = torch.zeros((2, 32), dtype=torch.bfloat16)
    qz, sz = olin.i8_quant_rows(z)
    assert int(qz.abs().sum()) == 0 and torch.allclose(sz, torch.full((2,), 1e-8))


def test_gemm_epilogue_matches_float64():
    x = inputs.outlier_activations(48, 256, seed=5)
    w, b = inputs.linear_weights(64, 256, w_seed=6, b_seed=7)
    qx, sx = olin.i8_quant_rows(x)
    qw, sw = olin.i8_quant_rows(w)
    y, acc = olin.i8_gemm(qx, qw, sx, sw, b)
    ref = (acc.double() * sx.double()[:, None] * sw.double()[None, :] + b.double()[None, :])
    assert torch.allclose(y.double(), ref, rtol=2 ** -8, atol=1e-6)
    g, _ = olin.i8_gemm(qx, qw, sx, sw, b, gelu=True)
    yd = y.double()
    closed = 0.5 * yd * (1 + torch.tanh(np.sqrt(2 / np.pi) * (yd + 0.044715 * yd ** 3)))
    assert torch.allclose(g.double(), closed, rtol=2 ** -7, atol=1e-6)


def test_int8_linear_close_to_bf16_linear():
    x, w, b = inputs.linear_1p3b()
    x, w = x[:256], w[:192]
    b = b[:192]
    y = olin.i8_linear(x, w, b).double()
    ref = x.double() @ w.double().t() + b.double()
    rel = (y - ref).norm() / ref.norm()
    # per-token int8 with x20 outlier channels: coarse steps on the other channels
    assert rel < 0.08, float(rel)


def test_fp8_reference_scales_and_codes():
    x, w, b = inputs.linear_1p3b()
    x = x[:128]
    w_fp8, w_scale = olin.fp8_quant_weight(w)
    assert w_scale.dtype == torch.float32
    assert w_scale == (w.float().abs().amax() / 448.0)
    x_fp8, a_scale = olin.fp8_quant_act(x)
    assert a_scale.dtype == torch.bfloat16  # bf16 arithmetic, as in the reference
    assert a_scale.float() == (x.float().abs().amax() / 448.0).to(torch.bfloat16).float()
    # the quotient is rounded to bf16 before the e4m3 cast
    q_bf16 = (x.float() / a_scale.float()).to(torch.bfloat16)
    assert torch.equal(x_fp8.view(torch.uint8), ofp8.encode(q_bf16))


def test_fp8_scaled_mm_matches_decoded_product():
    x, w, b = inputs.linear_1p3b()
    x, w, b = x[:64], w[:96], b[:96]
    w_fp8, w_scale = olin.fp8_quant_weight(w)
    y = olin.fp8_linear(x, w_fp8, w_scale, b)
    x_fp8, a_scale = olin.fp8_quant_act(x)
    ref = (x_fp8.double() @ w_fp8.double().t()) * float(a_scale) * float(w_scale) + b.double()
    assert torch.allclose(y.double(), ref, rtol=2 ** -7, atol=1e-4)


def test_fp32_quotient_equals_rounded_fp64_reciprocal_product():
    """The quantizers form x / s as RN32(RN64(x * RN64(1 / s))); for fp32 x and s this is the IEEE fp32
    quotient the oracle's torch division gives, also next to exact halfway points of the integer rounding."""
    rng = np.random.default_rng(7)
    n = 2_000_000
    amax = (rng.random(n, dtype=np.float32) * 100 + 1e-3).astype(np.float32)
    x = (rng.standard_normal(n).astype(np.float32) * amax / 3).astype(np.float32)
    x = (x.view(np.uint32) & 0xFFFF0000).view(np.float32)           # bf16 activations
    s = np.maximum(amax / np.float32(127), np.float32(1e-8)).astype(np.float32)
    cases = [(x, s)]
    k = rng.integers(-127, 127, n).astype(np.float32)
    s2 = (rng.random(n, dtype=np.float32) * 3 + 0.01).astype(np.float32)
    mid = ((k + np.float32(0.5)) * s2).astype(np.float32)
    for d in (-2, -1, 0, 1, 2):                                      # neighbours of k + 1/2 quotients
        cases.append(((mid.view(np.int32) + d).view(np.float32), s2))
    e4 = (rng.integers(-448, 449, n) / 8).astype(np.float32)        # e4m3-range quotients
    cases.append(((e4 * s2).astype(np.float32), s2))
    for xs, ss in cases:
        ref = (xs / ss).astype(np.float32)
        got = (xs.astype(np.float64) * (1.0 / ss.astype(np.float64))).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # a plain fp32 reciprocal product is not enough (so the check has teeth)
    xs, ss = cases[3]
    assert not np.array_equal((xs * (np.float32(1) / ss)).astype(np.float32), (xs / ss).astype(np.float32))
