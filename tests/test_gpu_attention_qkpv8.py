"""GPU parity of the paged attention with both products on the fp8 matrix cores (wf_attn_paged_fp8_qkpv8, the
``hip_fp8_qkpv`` backend: the counterpart of the fp8 P.V product of the reference's SageAttention backend,
wave_rt/runtime/backend.py:57-62,144-146).

The kernel is compared with the oracle of the same form (oracle.attention.paged_fp8_qkpv8, which forms the
e4m3 weights tile by tile as the kernel does) under the attention bar, |out - oracle| - margin <= 2e-2
(heavy-tailed K/V: 2e-2 * max(1, |oracle|)), over the exact kernel's cases.  The margin is the oracle's
bound on what weights lying within a relative 2^-15 of an e4m3 rounding midpoint can move an output by when
they round the other way: the kernel's fp32 scores (the matrix cores' own accumulation) and exponentials
(v_exp_f32) differ from the oracle's in the last bits, and near a midpoint that decides the rounding; one
such weight moves a row of a short context by up to a few percent.  Each query keeps its own lazy maximum in
the kernel as in the oracle, so any sample of rows can be passed to the oracle.  The distance from the exact attention (oracle.attention.paged_fp8) is printed
next to it: the approximation the form makes.
"""

import math

import pytest
import torch

from oracle import attention as oat
from oracle import kv as okv
from waveforcing_amd import _lib, inputs
from waveforcing_amd.backend import _WAVE_STATE, attend, attn_paged_fp8, attn_paged_fp8_qkpv, enable_hip_fp8, \
    enable_hip_fp8_qkpv
from waveforcing_amd.kv import Fp8PagePool, PagedKV

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-2
EPS = 2.0 ** -15    # rounding-midpoint band of the oracle's margin


def _excess(out, ref, margin, relative=False):
    d = (out - ref).abs() - margin
    return (d / ref.abs().clamp(min=1.0) if relative else d).max().item()


def _setup(Lq, H, n_kv, page, P, seed, heavy=False, k=None, v=None, q=None):
    if k is None:
        k = inputs.heavy_tailed_kv(n_kv, H, 128, seed=seed) if heavy else \
            torch.randn((n_kv, H, 128), generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
    if v is None:
        v = inputs.heavy_tailed_kv(n_kv, H, 128, seed=seed + 1) if heavy else \
            torch.randn((n_kv, H, 128), generator=torch.Generator().manual_seed(seed + 1)).to(torch.bfloat16)
    if q is None:
        q = torch.randn((Lq, H, 128), generator=torch.Generator().manual_seed(seed + 2)).to(torch.bfloat16)
    ids = inputs.page_table(-(-n_kv // page), P, seed=seed + 3)
    pool = Fp8PagePool(P, H, 128, page, DEV)
    table = pool.page_table(ids)
    pool.pack(k.to(DEV), v.to(DEV), table)
    kp, vp = okv.new_pool(P, page, H, 128), okv.new_pool(P, page, H, 128)
    okv.pack(k, ids, page, *kp)
    okv.pack(v, ids, page, *vp)
    return q, PagedKV(pool, table, n_kv), ids, kp, vp


def _oracle_blocks(q, blocks, kp, vp, ids, n_kv, page):
    """The oracle over row blocks [a, b) of q, concatenated."""
    return oat.paged_fp8_qkpv8(torch.cat([q[a:b] for a, b in blocks], 0), kp, vp, ids, n_kv, page, margin_eps=EPS)


@pytest.mark.parametrize("Lq,H,n_kv,page,P,seed", [
    (300, 2, 3 * 64 + 17, 80, 7, 0),     # ragged keys, small pages
    (130, 3, 64, 64, 2, 1),              # single tile, query tail
    (128, 12, 4680, 1560, 6, 2),         # one 1.3B chunk of context
    (257, 5, 1000, 1560, 3, 3),          # partial page
    (1, 1, 1, 64, 1, 4),                 # one query, one key
    (33, 2, 63, 64, 2, 5),               # one partial tile
    (65, 2, 65, 64, 3, 6),               # one key past the first tile, on the second page
    (512, 4, 128, 64, 4, 7),             # two full query tiles, two full key tiles, page = tile
])
def test_qkpv8_matches_oracle(Lq, H, n_kv, page, P, seed):
    q, ctx, ids, kp, vp = _setup(Lq, H, n_kv, page, P, seed)
    out = attn_paged_fp8(q.to(DEV).unsqueeze(0), ctx, fp8_pv=True).cpu()[0].float()
    ref, margin = oat.paged_fp8_qkpv8(q, kp, vp, ids, n_kv, page, margin_eps=EPS)
    exact = oat.paged_fp8(q, kp, vp, ids, n_kv, page)
    err, err_exact = (out - ref).abs().max().item(), (out - exact).abs().max().item()
    print(f"max abs err vs fp8-PV oracle {err:.3e} (beyond the rounding margin {_excess(out, ref, margin):.3e}); "
          f"vs exact attention {err_exact:.3e}")
    assert _excess(out, ref, margin) <= TOL


def test_qkpv8_heavy_tailed_relative():
    Lq, H, n_kv, page = 128, 12, 4680, 1560
    q, ctx, ids, kp, vp = _setup(Lq, H, n_kv, page, 6, seed=40, heavy=True)
    out = attn_paged_fp8_qkpv(q.to(DEV), ctx).cpu().float()
    ref, margin = oat.paged_fp8_qkpv8(q, kp, vp, ids, n_kv, page, margin_eps=EPS)
    exact = oat.paged_fp8(q, kp, vp, ids, n_kv, page)
    rel = _excess(out, ref, margin, relative=True)
    rel_exact = ((out - exact).abs() / exact.abs().clamp(min=1.0)).max().item()
    print(f"max rel err vs fp8-PV oracle beyond the rounding margin {rel:.3e}; vs exact attention {rel_exact:.3e}")
    assert rel <= TOL


@pytest.mark.parametrize("H,seed", [(12, 10), (40, 50)])
def test_qkpv8_full_context_sampled_waves(H, seed):
    """4680 queries over 8 chunks (37440 keys); five blocks of rows (the first 64, the partial last wave, two
    32-row waves drawn at random and 19 rows straddling two waves), all heads."""
    Lq, n_kv, page = 4680, 37440, 1560
    q, ctx, ids, kp, vp = _setup(Lq, H, n_kv, page, 26 if H == 40 else 30, seed=seed)
    out = attn_paged_fp8_qkpv(q.to(DEV), ctx).cpu().float()
    picks = torch.randperm(Lq // 32 - 3, generator=torch.Generator().manual_seed(seed))[:2] + 2
    blocks = [(0, 64)] + [(32 * int(w), 32 * int(w) + 32) for w in picks] + [(2000, 2019), (Lq // 32 * 32, Lq)]
    ref, margin = _oracle_blocks(q, blocks, kp, vp, ids, n_kv, page)
    got = torch.cat([out[a:b] for a, b in blocks], 0)
    exact = oat.paged_fp8(torch.cat([q[a:b] for a, b in blocks], 0), kp, vp, ids, n_kv, page)
    err, err_exact = (got - ref).abs().max().item(), (got - exact).abs().max().item()
    print(f"max abs err vs fp8-PV oracle {err:.3e} (beyond the rounding margin {_excess(got, ref, margin):.3e}); "
          f"vs exact attention {err_exact:.3e}")
    assert _excess(got, ref, margin) <= TOL


def _round_mantissa3(x: float) -> float:
    """x > 0 rounded to 4 significant bits (e4m3's normal precision), ties to even."""
    m, e = math.frexp(x)                 # x = m 2^e, m in [0.5, 1)
    r = m * 16.0
    n = math.floor(r)
    if r - n > 0.5 or (r - n == 0.5 and n % 2 == 1):
        n += 1
    return math.ldexp(n / 16.0, e)


def test_qkpv8_single_key_returns_its_weight_rounded_value():
    """One key and zero queries (score 0, so p = 1 exactly): the weight is s_v alone, carried with 4
    significant bits, so out = round4(s_v) * code_v."""
    H, Lq = 3, 40
    q, ctx, ids, kp, vp = _setup(Lq, H, 1, 64, 2, seed=90, q=torch.zeros((Lq, 3, 128), dtype=torch.bfloat16))
    out = attn_paged_fp8_qkpv(q.to(DEV), ctx).cpu().float()
    vc, vs = okv.gather(ids, 1, 64, *vp)
    for h in range(H):
        want = vc[0, h].view(okv.FP8).float() * _round_mantissa3(float(vs[0, h]))
        want = want.to(torch.bfloat16).float()
        assert torch.equal(out[:, h], want[None, :].expand(Lq, -1)), h


def test_qkpv8_equal_scores_with_power_of_two_scales_give_the_mean_of_v():
    """Zero queries score every key 0, so p = 1 for all keys; with V rows whose scales are powers of two every
    weight is exact in e4m3 and the output is the mean of V."""
    H, Lq, n_kv, page = 2, 64, 700, 128
    g = torch.Generator().manual_seed(91)
    codes = torch.randint(0, 126, (n_kv, H, 128), generator=g, dtype=torch.uint8)
    codes[:, :, 0] = 126                                        # e4m3 448: the row maximum
    signs = torch.randint(0, 2, (n_kv, H, 128), generator=g, dtype=torch.uint8) << 7
    vals = (codes | signs).view(okv.FP8).float()
    pw = torch.randint(-8, -1, (n_kv, H, 1), generator=g).float()
    v = (vals * torch.pow(2.0, pw)).to(torch.bfloat16)
    q = torch.zeros((Lq, H, 128), dtype=torch.bfloat16)
    q_, ctx, ids, kp, vp = _setup(Lq, H, n_kv, page, 8, seed=92, v=v, q=q)
    assert torch.all(torch.log2(okv.gather(ids, n_kv, page, *vp)[1]).frac() == 0)
    out = attn_paged_fp8_qkpv(q.to(DEV), ctx).cpu().float()
    want = v.double().mean(dim=0).to(torch.bfloat16).float()[None]
    err = ((out - want).abs() / want.abs().clamp(min=2 ** -10)).max().item()
    print(f"mean of V: max rel err {err:.3e}")
    assert err <= 2 ** -7                                     # within a bf16 step


def test_qkpv8_invalid_page_ids_read_as_zero_keys():
    """As for the exact form: table entries outside the pool read as zero codes and zero scales."""
    Lq, H, page, P = 96, 3, 200, 6
    n_kv = 4 * page + 77
    gen = lambda shape, s: torch.randn(shape, generator=torch.Generator().manual_seed(s)).to(torch.bfloat16)
    k, v, q = gen((n_kv, H, 128), 70), gen((n_kv, H, 128), 71), gen((Lq, H, 128), 72)
    ids = [4, 0, 5, 2, 1]
    pool = Fp8PagePool(P, H, 128, page, DEV)
    pool.pack(k.to(DEV), v.to(DEV), pool.page_table(ids))
    bad = list(ids)
    bad[1], bad[3] = -1, P
    table = torch.tensor(bad, dtype=torch.int32, device=DEV)
    qd = q.to(DEV)
    out = torch.empty((Lq, H, 128), dtype=torch.bfloat16, device=DEV)
    _lib.call("wf_attn_paged_fp8_qkpv8", qd.data_ptr(), Lq, H, 128, qd.stride(0), pool.k_codes.data_ptr(),
              pool.v_codes.data_ptr(), pool.k_scales.data_ptr(), pool.v_scales.data_ptr(), P, page, table.data_ptr(),
              len(bad), n_kv, 1.0 / math.sqrt(128), out.data_ptr(), out.stride(0), _lib.stream_handle(DEV))
    kc, ks = okv.quantize_rows(k)
    vc, vs = okv.quantize_rows(v)
    for lp in (1, 3):
        rows = slice(lp * page, (lp + 1) * page)
        kc[rows], ks[rows], vc[rows], vs[rows] = 0, 0.0, 0, 0.0
    ref, margin = oat.sdpa_qkpv8(q, kc, ks, vc, vs, margin_eps=EPS)
    err = _excess(out.cpu().float(), ref, margin)
    print(f"max abs err beyond the rounding margin {err:.3e}")
    assert err <= TOL, err


def test_backend_dispatch_selects_fp8_pv():
    q, ctx, ids, kp, vp = _setup(64, 2, 128, 64, 3, seed=80)
    saved = dict(_WAVE_STATE)
    try:
        enable_hip_fp8_qkpv()
        assert _WAVE_STATE["attn"] == "hip_fp8_qkpv"
        got = attend(q.to(DEV).unsqueeze(0), ctx, ctx).cpu()[0]
        want = attn_paged_fp8(q.to(DEV), ctx, fp8_pv=True).cpu()
        assert torch.equal(got, want)
        enable_hip_fp8()
        assert torch.equal(attend(q.to(DEV).unsqueeze(0), ctx, ctx).cpu()[0], attn_paged_fp8(q.to(DEV), ctx).cpu())
    finally:
        _WAVE_STATE.clear()
        _WAVE_STATE.update(saved)
