"""Pins the FP8 KV oracle (oracle/kv.py) without the GPU.

Checks that would fail for a plausible mistake in the restatement:
- scale closed form: rows whose amax is 448 * 2^k get scale exactly 2^k;
- the largest-|x| element of every row encodes to +-448 (a wrong divisor,
  e.g. 127, or a missing scale breaks it);
- the bf16 rounding of the scale (common.py:146-148 divides in bf16) is
  observable on the golden inputs: an fp32 scale gives different codes;
- round-trip error within half an e4m3 step (plus the bf16 output rounding);
- the identity page table over contiguous pages equals the plain
  concatenation of the rows (paging changes layout, not numbers);
- a shuffled page table puts each token block in its page (brute force), and
  pages not in the table stay untouched;
- the committed golden fixture.
"""

import os

import numpy as np
import torch

from oracle import fp8 as ofp8
from oracle import kv as okv
from waveforcing_amd import inputs

GOLD = os.path.join(os.path.dirname(__file__), "golden", "kv_small.npz")


def test_scale_closed_form_power_of_two():
    g = torch.Generator().manual_seed(0)
    rows = torch.rand((64, 128), generator=g) * 2 - 1
    k = torch.arange(64) % 9 - 4  # scales 2^-4 .. 2^4
    rows[:, 7] = 1.0
    rows = rows * (448.0 * torch.pow(2.0, k.float()))[:, None]
    rows = rows.to(torch.bfloat16)
    codes, scales = okv.quantize_rows(rows)
    assert torch.equal(scales, torch.pow(2.0, k.float()))
    exact = ofp8.encode((rows.float() / scales[:, None]))
    assert torch.equal(codes, exact)


def test_row_max_encodes_to_448():
    x = inputs.heavy_tailed_kv(300, 4, 128, seed=5)
    codes, _ = okv.quantize_rows(x)
    idx = x.float().abs().argmax(-1, keepdim=True)
    top = torch.gather(codes, -1, idx).squeeze(-1)
    assert bool(((top == 0x7E) | (top == 0xFE)).all())


def test_scale_is_rounded_to_bf16():
    g = np.load(GOLD)
    k = torch.from_numpy(g["k_bits"]).view(torch.bfloat16)
    codes, scales = okv.quantize_rows(k)
    s32 = (k.float().abs().amax(-1, keepdim=True) / 448.0).clamp(min=1e-8)
    wrong = ofp8.encode((k.float() / s32).clamp(-448, 448))
    assert not torch.equal(wrong, codes)
    assert torch.equal(scales.to(torch.bfloat16).float(), scales)


def test_roundtrip_error_bound():
    x = inputs.heavy_tailed_kv(500, 3, 128, seed=9)
    codes, scales = okv.quantize_rows(x)
    deq = okv.dequantize_rows(codes, scales).double()
    xf = x.double()
    s = scales.double()[..., None]
    q = xf / s
    step = torch.where(q.abs() >= 2.0 ** -6, q.abs() * 2.0 ** -4, torch.full_like(q, 2.0 ** -10))
    bound = step * s + deq.abs() * 2.0 ** -8 + 1e-30
    assert bool(((deq - xf).abs() <= bound).all())


def test_identity_table_equals_concatenation():
    T, H, D, page = 4680, 2, 128, 1560
    x = inputs.heavy_tailed_kv(T, H, D, seed=3)
    cp, sp = okv.new_pool(3, page, H, D)
    okv.pack(x, [0, 1, 2], page, cp, sp)
    codes, scales = okv.quantize_rows(x)
    assert torch.equal(cp.reshape(T, H, D), codes)
    assert torch.equal(sp.transpose(1, 2).reshape(T, H), scales)
    assert torch.equal(okv.unpack([0, 1, 2], T, page, cp, sp), okv.dequantize_rows(codes, scales))


def test_shuffled_table_brute_force():
    T, H, D, page, P = 37, 3, 128, 8, 9
    x = inputs.heavy_tailed_kv(T, H, D, seed=4)
    table = [6, 2, 8, 0, 5]
    cp, sp = okv.new_pool(P, page, H, D)
    okv.pack(x, table, page, cp, sp)
    codes, scales = okv.quantize_rows(x)
    for t in range(T):
        p, r = table[t // page], t % page
        for h in range(H):
            assert torch.equal(cp[p, r, h], codes[t, h])
            assert sp[p, h, r] == scales[t, h]
    untouched = [p for p in range(P) if p not in table]
    assert int(cp[untouched].abs().sum()) == 0 and float(sp[untouched].abs().sum()) == 0.0
    # rows past T in the last page stay zero
    assert int(cp[table[-1], T % page:].abs().sum()) == 0


def test_golden_fixture():
    g = np.load(GOLD)
    k = torch.from_numpy(g["k_bits"]).view(torch.bfloat16)
    v = torch.from_numpy(g["v_bits"]).view(torch.bfloat16)
    page, P = int(g["page_tokens"]), int(g["pool_pages"])
    table = g["table"].tolist()
    kc, ks = okv.new_pool(P, page, k.shape[1], k.shape[2])
    vc, vs = okv.new_pool(P, page, k.shape[1], k.shape[2])
    okv.pack(k, table, page, kc, ks)
    okv.pack(v, table, page, vc, vs)
    assert np.array_equal(kc.numpy(), g["k_codes"]) and np.array_equal(ks.numpy(), g["k_scales"])
    assert np.array_equal(vc.numpy(), g["v_codes"]) and np.array_equal(vs.numpy(), g["v_scales"])
    # the zero row takes the scale floor bf16(1e-8) and all-zero codes
    assert ks[table[0], 0, 0].item() == torch.tensor(1e-8).to(torch.bfloat16).float().item()


# ---- per-tensor FP8 KV (common.py:143-164)
def test_pertensor_codes_and_scale_equal_the_pinned_activation_quantizer():
    from oracle import linear as olin
    kv = inputs.heavy_tailed_kv(96, 3, 128, seed=21)
    codes, scale = okv.quantize_tensor(kv)
    want_codes, want_scale = olin.fp8_quant_act(kv.reshape(-1, 128))
    assert torch.equal(codes.reshape(-1, 128), want_codes.view(torch.uint8))
    assert scale.shape == (1,) and float(scale) == float(want_scale)


def test_pertensor_dtypes_and_closed_forms():
    # amax = 448 * 2^-3: the scale is exactly 2^-3, and the row max encodes to 448 (0x7e)
    kv = torch.zeros((2, 4, 1, 128), dtype=torch.bfloat16)
    kv[0, 1, 0, 5] = 56.0
    kv[1, 2, 0, 7] = -1.5
    codes, scale = okv.quantize_tensor(kv)
    assert scale.dtype == torch.float32 and float(scale) == 0.125
    assert int(codes[0, 1, 0, 5]) == 0x7E and int(codes[1, 2, 0, 7]) == 0xD4   # -12: sign, exponent 3 + 7, mantissa .100
    deq = okv.dequantize_tensor(codes, scale)
    assert deq.dtype == torch.float32                  # the reference's dequant is fp32 by promotion
    assert float(deq[0, 1, 0, 5]) == 56.0 and float(deq[1, 2, 0, 7]) == -1.5
    # the scale is amax / 448 rounded to bf16: amax 1 gives bf16(1/448), not the fp32 quotient
    one = torch.zeros((1, 1, 1, 128), dtype=torch.bfloat16)
    one[0, 0, 0, 0] = 1.0
    s = float(okv.quantize_tensor(one)[1])
    assert s == float(torch.tensor(1 / 448, dtype=torch.float32).to(torch.bfloat16)) and s != float(
        torch.tensor(1.0 / 448.0, dtype=torch.float32))
    # an all-zero tensor takes the bf16 floor of 1e-8 (bits 0x322c)
    z, zs = okv.quantize_tensor(torch.zeros((1, 2, 1, 128), dtype=torch.bfloat16))
    assert int(z.abs().sum()) == 0
    assert torch.tensor([float(zs)]).to(torch.bfloat16).view(torch.int16).item() == 0x322C


def test_pertensor_quotient_is_rounded_to_bf16_before_the_cast():
    """x / s is rounded to bf16 first: pick x, s where the fp32 quotient and its bf16 rounding encode to
    different e4m3 codes, and check the oracle gives the code of the bf16-rounded quotient."""
    s = 0.125 * (1 + 2 ** -7)                               # a bf16 scale (amax = 448 * s)
    found = 0
    for m in range(128, 256):
        x = torch.tensor([m * 2.0 ** -7 * 1.25], dtype=torch.float32).to(torch.bfloat16)
        q32 = x.float() / torch.tensor(s)
        qb = q32.to(torch.bfloat16).float()
        c32 = int(q32.to(okv.FP8).view(torch.uint8))
        cb = int(qb.to(okv.FP8).view(torch.uint8))
        if c32 == cb:
            continue
        kv = torch.zeros((1, 1, 1, 128), dtype=torch.bfloat16)
        kv[0, 0, 0, 0] = torch.tensor(448 * s).to(torch.bfloat16)
        kv[0, 0, 0, 1] = x
        codes, scale = okv.quantize_tensor(kv)
        assert float(scale) == s
        assert int(codes[0, 0, 0, 1]) == cb
        found += 1
    assert found > 0
