"""Pins the e4m3fn codec oracle (torch's cast) without the GPU.

Checks: an independent nearest-value encoder over every bf16 bit pattern and
every fp32 value next to a rounding boundary; the closed-form decode of all
256 codes; known answers at the saturation and subnormal edges; the committed
golden tables.
"""

import os

import numpy as np
import torch

from oracle import fp8 as ofp8

GOLD = os.path.join(os.path.dirname(__file__), "golden", "e4m3_tables.npz")


def test_torch_cast_equals_independent_encoder_on_all_bf16():
    x = ofp8.all_bf16_as_f32()
    ref = ofp8.encode(x).numpy()
    ind = ofp8.encode_bits(x.numpy())
    assert np.array_equal(ref, ind)


def test_torch_cast_equals_independent_encoder_at_boundaries():
    x = ofp8.boundary_f32()
    assert x.numel() > 2000
    assert np.array_equal(ofp8.encode(x).numpy(), ofp8.encode_bits(x.numpy()))


def test_decode_matches_closed_form():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    got = ofp8.decode(codes).numpy().astype(np.float64)
    want = ofp8.decode_closed_form(np.arange(256))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    assert np.isnan(want).sum() == 2  # only 0x7f and 0xff


def test_known_answers():
    cases = [
        (448.0, 0x7E), (449.0, 0x7E), (464.0, 0x7E),  # 464 ties to even (448)
        (464.03125, 0x7F), (480.0, 0x7F), (float("inf"), 0x7F), (float("nan"), 0x7F),
        (-448.0, 0xFE), (-500.0, 0xFF), (-0.0, 0x80), (0.0, 0x00),
        (2.0 ** -9, 0x01), (2.0 ** -10, 0x00),  # half the smallest subnormal ties to 0
        (1.5 * 2.0 ** -9, 0x02), (2.5 * 2.0 ** -9, 0x02),  # ties to even
        (2.0 ** -6, 0x08), (1.0, 0x38), (1.0625, 0x38), (1.0625001, 0x39), (1.1875, 0x3A),
        (-1e-30, 0x80),
    ]
    x = torch.tensor([c[0] for c in cases], dtype=torch.float32)
    got = ofp8.encode(x).tolist()
    assert got == [c[1] for c in cases]


def test_golden_tables():
    g = np.load(GOLD)
    assert np.array_equal(g["enc_bf16"], ofp8.encode(ofp8.all_bf16_as_f32()).numpy())
    dec = ofp8.decode(torch.arange(256, dtype=torch.int32).to(torch.uint8)).numpy()
    assert np.array_equal(np.isnan(g["dec"]), np.isnan(dec))
    assert np.array_equal(np.nan_to_num(g["dec"]), np.nan_to_num(dec))
