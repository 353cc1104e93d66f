"""Pins the attention oracle (oracle/attention.py) on the CPU.

Closed forms: constant V returns V; a single key returns its V row;
identical keys give the mean of V; a zero scale gives the mean of V; key
order does not matter; and a float64 numpy evaluation of the definition
agrees on random data.  The paged path equals attention over the plain
concatenation of the dequantized rows (paging changes layout only).

The quantized-QK form (paged_fp8_qk8): queries whose rows are already e4m3
values times a power of two (amax = 448 * 2^k) pass the quantization
unchanged, so the form reduces to the exact paged attention; a single key
returns its V row; all-zero queries give the mean of V; each query row's
scale is the smallest power of two with amax <= 448 s_q, so its largest code
lies in [224, 448], and every code is the e4m3 rounding of q / s_q (ties to
even, checked on exact ties); and on N(0, 1) data the form stays within the
attention bar of the exact one while differing from it.
"""

import math

import numpy as np
import torch

from oracle import attention as oat
from oracle import kv as okv
from waveforcing_amd import inputs


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16)


def test_matches_float64_definition():
    q, k, v = _rand((17, 3, 128), 0), _rand((45, 3, 128), 1), _rand((45, 3, 128), 2)
    got = oat.sdpa(q, k, v).double().numpy()
    qd, kd, vd = (t.double().numpy() for t in (q, k, v))
    want = np.zeros_like(got)
    for h in range(3):
        s = qd[:, h] @ kd[:, h].T / math.sqrt(128)
        e = np.exp(s - s.max(-1, keepdims=True))
        want[:, h] = (e / e.sum(-1, keepdims=True)) @ vd[:, h]
    assert np.abs(got - want).max() < 1e-5


def test_closed_forms():
    q, k = _rand((9, 2, 128), 3), _rand((30, 2, 128), 4)
    vrow = _rand((1, 2, 128), 5)
    const_v = vrow.expand(30, 2, 128)
    assert torch.allclose(oat.sdpa(q, k, const_v), vrow.float().expand(9, 2, 128), atol=1e-5)
    one = oat.sdpa(q, k[:1], _rand((1, 2, 128), 6))
    assert torch.allclose(one, _rand((1, 2, 128), 6).float().expand(9, 2, 128), atol=1e-6)
    v = _rand((30, 2, 128), 7)
    same_k = k[:1].expand(30, 2, 128)
    assert torch.allclose(oat.sdpa(q, same_k, v), v.float().mean(0, keepdim=True).expand(9, 2, 128), atol=1e-5)
    assert torch.allclose(oat.sdpa(q, k, v, scale=0.0), v.float().mean(0, keepdim=True).expand(9, 2, 128),
                          atol=1e-5)
    perm = torch.randperm(30, generator=torch.Generator().manual_seed(8))
    assert torch.allclose(oat.sdpa(q, k[perm], v[perm]), oat.sdpa(q, k, v), atol=1e-5)


def test_paged_equals_concatenated():
    T, H, page = 200, 2, 64
    k, v = inputs.heavy_tailed_kv(T, H, 128, 9), inputs.heavy_tailed_kv(T, H, 128, 10)
    q = _rand((20, H, 128), 11)
    table = [4, 1, 3, 0]
    kc, ks = okv.new_pool(5, page, H, 128)
    vc, vs = okv.new_pool(5, page, H, 128)
    okv.pack(k, table, page, kc, ks)
    okv.pack(v, table, page, vc, vs)
    got = oat.paged_fp8(q, (kc, ks), (vc, vs), table, T, page)
    ck, sk = okv.quantize_rows(k)
    cv, sv = okv.quantize_rows(v)
    want = oat.sdpa(q, okv.dequantize_rows(ck, sk), okv.dequantize_rows(cv, sv))
    assert torch.equal(got, want)


def _pool_of(k, v, page):
    n = k.shape[0]
    pages = -(-n // page)
    ids = list(range(pages))[::-1]
    kp, vp = okv.new_pool(pages, page, k.shape[1], 128), okv.new_pool(pages, page, k.shape[1], 128)
    okv.pack(k, ids, page, *kp)
    okv.pack(v, ids, page, *vp)
    return kp, vp, ids


def _e4m3_rows(n, heads, seed, pow2):
    """bf16 [n, heads, 128] rows of random e4m3 values whose amax is 448, times 2^pow2 (exact in bf16)."""
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 256, (n, heads, 128), generator=g, dtype=torch.uint8)
    vals = codes.view(okv.FP8).float()
    vals = torch.where(torch.isnan(vals), torch.zeros_like(vals), vals)
    vals[:, :, 0] = 448.0
    return (vals * 2.0 ** pow2).to(torch.bfloat16)


def test_qk8_reduces_to_exact_form_on_representable_queries():
    # queries and keys whose rows are e4m3 values times a power of two: the query codes are the rows
    # themselves and the K scale is a power of two, so code * s_k is also the exact form's bf16 K
    q = _e4m3_rows(40, 2, 11, -9)
    k, v = _e4m3_rows(150, 2, 12, -8), _rand((150, 2, 128), 13)
    kp, vp, ids = _pool_of(k, v, 64)
    qc, sq = oat.quantize_q_rows(q)
    assert torch.equal(qc * sq[..., None], q.float())
    got = oat.paged_fp8_qk8(q, kp, vp, ids, 150, 64)
    want = oat.paged_fp8(q, kp, vp, ids, 150, 64)
    assert (got - want).abs().max().item() < 1e-4


def test_qk8_closed_forms_and_error_scale():
    k, v = _rand((1, 3, 128), 14), _rand((1, 3, 128), 15)
    q = _rand((5, 3, 128), 16)
    kp, vp, ids = _pool_of(k, v, 64)
    one = oat.paged_fp8_qk8(q, kp, vp, ids, 1, 64)
    assert torch.equal(one, okv.unpack(ids, 1, 64, *vp).float().expand(5, 3, 128))
    k, v = _rand((200, 3, 128), 17), _rand((200, 3, 128), 18)
    kp, vp, ids = _pool_of(k, v, 64)
    zero = oat.paged_fp8_qk8(torch.zeros((4, 3, 128), dtype=torch.bfloat16), kp, vp, ids, 200, 64)
    mean = okv.unpack(ids, 200, 64, *vp).double().mean(0).float()
    assert (zero - mean).abs().max().item() < 1e-6
    # power-of-two scales: the smallest with amax <= 448 s_q, so every row's largest value lies in (224, 448] s_q
    # (its code in [224, 448] after rounding), and codes within half an e4m3 step (2^-4 relative) of q / s_q
    q = _rand((64, 3, 128), 19)
    qc, sq = oat.quantize_q_rows(q)
    mant, _ = torch.frexp(sq)
    assert (mant == 0.5).all()
    row_max = qc.abs().amax(dim=-1)
    assert ((row_max >= 224.0) & (row_max <= 448.0)).all()
    assert (q.float().abs().amax(dim=-1) <= 448.0 * sq).all() and (q.float().abs().amax(dim=-1) > 224.0 * sq).all()
    ideal = q.float() / sq[..., None]
    assert ((qc - ideal).abs() <= ideal.abs() * 2.0 ** -4 + 2.0 ** -10).all()
    # amax 3 takes s_q = 2^-7 (3 * 2^7 = 384 <= 448 < 768); 1.0625 * 2^7 = 136 is an e4m3 tie between 128 and 144
    # and 1.1875 * 2^7 = 152 one between 144 and 160: ties go to the even code (128, 160); amax 448 keeps s_q = 1
    tie = torch.zeros((1, 1, 128), dtype=torch.bfloat16)
    tie[0, 0, 0], tie[0, 0, 1], tie[0, 0, 2] = 3.0, 1.0625, 1.1875
    tc, ts = oat.quantize_q_rows(tie)
    assert float(ts[0, 0]) == 2.0 ** -7 and tc[0, 0, :3].tolist() == [384.0, 128.0, 160.0]
    top = torch.zeros((1, 1, 128), dtype=torch.bfloat16)
    top[0, 0, 5] = -448.0
    tc, ts = oat.quantize_q_rows(top)
    assert float(ts[0, 0]) == 1.0 and float(tc[0, 0, 5]) == -448.0
    got = oat.paged_fp8_qk8(q, kp, vp, ids, 200, 64)
    exact = oat.paged_fp8(q, kp, vp, ids, 200, 64)
    err = (got - exact).abs().max().item()
    assert 0 < err < 2e-2


# ---- the fp8-PV form (oracle.attention.sdpa_qkpv8) ----------------------------------------------------------------

def _codes_and_scales(x):
    return okv.quantize_rows(x)


def _exact_v(vc, vs):
    return vc.view(okv.FP8).float() * vs[..., None]


def test_qkpv8_without_weight_rounding_is_the_quantized_qk_form():
    """With the weights left unrounded the tile-by-tile evaluation (each query's lazy maximum, rescaled sums,
    masked tail keys) must give the quantized-QK attention of the definition over V = code * s.
    Later tiles carry keys scaled up 3x per tile, so the running maxima move by far more than the rescale
    threshold and the rescale path runs."""
    for Lq, H, n, seed in ((70, 2, 200, 0), (33, 1, 64, 1), (5, 1, 65, 2), (100, 2, 1, 3), (40, 1, 300, 4)):
        q, k, v = _rand((Lq, H, 128), seed), _rand((n, H, 128), seed + 10), _rand((n, H, 128), seed + 20)
        if seed == 4:
            grow = torch.pow(3.0, (torch.arange(n) // 64).float())[:, None, None]
            k = (k.float() * grow).to(torch.bfloat16)
        kc, ks = _codes_and_scales(k)
        vc, vs = _codes_and_scales(v)
        got = oat.sdpa_qkpv8(q, kc, ks, vc, vs, round_p=False)
        want = oat.sdpa_qk8(q, kc, ks, _exact_v(vc, vs))
        assert (got - want).abs().max().item() < 1e-4, (Lq, H, n)    # fp32 exponents against float64 ones
        rounded = oat.sdpa_qkpv8(q, kc, ks, vc, vs)
        assert 0 < (rounded - want).abs().max().item() < 0.2


def test_qkpv8_rows_are_independent():
    """Each query keeps its own lazy maximum, as the kernel does: rows evaluated alone, or in another order,
    give the same values as in one call.  Keys grow 3x per tile and every other query is scaled down 64x, so
    the rescale path runs for the large queries while the small ones keep their maxima."""
    Lq, H, n = 45, 2, 300
    q, k, v = _rand((Lq, H, 128), 50), _rand((n, H, 128), 51), _rand((n, H, 128), 52)
    q = (q.float() * torch.where(torch.arange(Lq) % 2 == 0, 1.0, 1.0 / 64)[:, None, None]).to(torch.bfloat16)
    k = (k.float() * torch.pow(3.0, (torch.arange(n) // 64).float())[:, None, None]).to(torch.bfloat16)
    kc, ks = _codes_and_scales(k)
    vc, vs = _codes_and_scales(v)
    full = oat.sdpa_qkpv8(q, kc, ks, vc, vs)
    perm = torch.randperm(Lq, generator=torch.Generator().manual_seed(53))
    assert torch.equal(oat.sdpa_qkpv8(q[perm], kc, ks, vc, vs), full[perm])
    for r in (0, 17, 44):
        assert torch.equal(oat.sdpa_qkpv8(q[r:r + 1], kc, ks, vc, vs)[0], full[r])


def _round4(x: float) -> float:
    """x > 0 to 4 significant bits, ties to even (e4m3's normal precision)."""
    m, e = math.frexp(x)
    r = m * 16.0
    n = math.floor(r)
    if r - n > 0.5 or (r - n == 0.5 and n % 2 == 1):
        n += 1
    return math.ldexp(n / 16.0, e)


def test_qkpv8_single_key_carries_its_scale_with_four_significant_bits():
    """Zero queries over one key: p = 1, the weight is s_v itself, rounded to 4 significant bits (ties to even):
    out = round4(s_v) * code_v.  Scales with significands 1, 1.0625 (a tie, to 1), 1.09375 (to 1.125),
    1.75, 1.875 and 1.9921875 (to 2) at several powers of two."""
    for f in (1.0, 1.0625, 1.09375, 1.75, 1.875, 1.9921875):
        for j in (-12, -7, 0, 3):
            v = _rand((1, 1, 128), 30) * 0.01
            v[0, 0, 7] = 448.0 * f * 2.0 ** j
            vc, vs = _codes_and_scales(v)
            assert float(vs[0, 0]) == f * 2.0 ** j
            kc, ks = _codes_and_scales(_rand((1, 1, 128), 31))
            got = oat.sdpa_qkpv8(torch.zeros((3, 1, 128), dtype=torch.bfloat16), kc, ks, vc, vs)
            want = vc[0, 0].view(okv.FP8).float() * _round4(f * 2.0 ** j)
            assert torch.equal(got[:, 0], want[None].expand(3, 128)), (f, j)


def test_qkpv8_equal_scores_with_power_of_two_scales_give_the_mean_of_v():
    g = torch.Generator().manual_seed(32)
    n = 300
    codes = torch.randint(0, 126, (n, 2, 128), generator=g, dtype=torch.uint8)
    codes[:, :, 0] = 126
    vals = codes.view(okv.FP8).float() * torch.where(torch.rand((n, 2, 128), generator=g) < 0.5, -1.0, 1.0)
    v = (vals * torch.pow(2.0, torch.randint(-9, 0, (n, 2, 1), generator=g).float())).to(torch.bfloat16)
    vc, vs = _codes_and_scales(v)
    kc, ks = _codes_and_scales(_rand((n, 2, 128), 33))
    got = oat.sdpa_qkpv8(torch.zeros((5, 2, 128), dtype=torch.bfloat16), kc, ks, vc, vs)
    want = v.double().mean(0)
    assert (got.double() - want[None]).abs().max().item() < 1e-6


def test_pv8_exponent_rule():
    mx = torch.tensor([448.0, 448.5, 224.0, 224.5, 256.0, 1.0, 0.0, 2.0 ** -200, 1e38], dtype=torch.float64)
    assert oat.pv8_exponent(mx).tolist() == [0, 1, -1, 0, 0, -8, 0, -126, 118]
    e = oat.pv8_exponent(mx[:6]).double()
    assert ((mx[:6] <= 448 * torch.pow(2.0, e)) & (mx[:6] > 448 * torch.pow(2.0, e - 1))).all()
