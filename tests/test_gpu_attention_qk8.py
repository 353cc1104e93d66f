"""GPU parity of the quantized-QK paged attention (wf_attn_paged_fp8_qk8, the
``hip_fp8_qk`` backend: the counterpart of the reference's SageAttention
backend, wave_rt/runtime/backend.py:57-62,144-146).

The kernel is compared with the oracle of the same form
(oracle.attention.paged_fp8_qk8: per-row e4m3 queries, the pages' K codes,
scores times s_q * s_k, exact V) under the attention bar, max |out - oracle|
<= 2e-2 (heavy-tailed K/V: 2e-2 * max(1, |oracle|)), over the exact kernel's
cases.  Its distance from the exact attention (oracle.attention.paged_fp8)
is printed next to it: that is the approximation the form makes, as Sage's
int8 QK does.  On rows that are e4m3 values times a power of two the form
equals the exact attention, and the kernel must then agree with the exact
kernel.
"""

import pytest
import torch

from oracle import attention as oat
from oracle import kv as okv
from waveforcing_amd import inputs
from waveforcing_amd.backend import _WAVE_STATE, attend, attn_paged_fp8, attn_paged_fp8_qk, enable_hip_fp8, \
    enable_hip_fp8_qk
from waveforcing_amd.kv import Fp8PagePool, PagedKV

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-2


def _setup(Lq, H, n_kv, page, P, seed, heavy=False, k=None, q=None):
    if k is None:
        k = inputs.heavy_tailed_kv(n_kv, H, 128, seed=seed) if heavy else \
            torch.randn((n_kv, H, 128), generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
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


def _errors(out, q, ids, kp, vp, n_kv, page, rows=None):
    qs = q if rows is None else q[rows]
    o = out.float() if rows is None else out[rows].float()
    ref = oat.paged_fp8_qk8(qs, kp, vp, ids, n_kv, page)
    exact = oat.paged_fp8(qs, kp, vp, ids, n_kv, page)
    return (o - ref).abs().max().item(), (o - exact).abs().max().item(), ref


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
def test_qk8_matches_quantized_qk_oracle(Lq, H, n_kv, page, P, seed):
    q, ctx, ids, kp, vp = _setup(Lq, H, n_kv, page, P, seed)
    out = attn_paged_fp8(q.to(DEV).unsqueeze(0), ctx, quantized_qk=True).cpu()[0]
    err, err_exact, _ = _errors(out, q, ids, kp, vp, n_kv, page)
    print(f"max abs err vs quantized-QK oracle {err:.3e}; vs exact attention {err_exact:.3e}")
    assert err <= TOL


def test_qk8_heavy_tailed_relative():
    Lq, H, n_kv, page = 128, 12, 4680, 1560
    q, ctx, ids, kp, vp = _setup(Lq, H, n_kv, page, 6, seed=40, heavy=True)
    out = attn_paged_fp8_qk(q.to(DEV), ctx).cpu().float()
    ref = oat.paged_fp8_qk8(q, kp, vp, ids, n_kv, page)
    exact = oat.paged_fp8(q, kp, vp, ids, n_kv, page)
    rel = ((out - ref).abs() / ref.abs().clamp(min=1.0)).max().item()
    rel_exact = ((out - exact).abs() / exact.abs().clamp(min=1.0)).max().item()
    print(f"max rel err vs quantized-QK oracle {rel:.3e}; vs exact attention {rel_exact:.3e}")
    assert rel <= TOL


@pytest.mark.parametrize("H,seed", [(12, 10), (40, 50)])
def test_qk8_full_context_sampled_rows(H, seed):
    """4680 queries over 8 chunks (37440 keys); 160 sampled rows, all heads."""
    Lq, n_kv, page = 4680, 37440, 1560
    q, ctx, ids, kp, vp = _setup(Lq, H, n_kv, page, 26 if H == 40 else 30, seed=seed)
    out = attn_paged_fp8_qk(q.to(DEV), ctx).cpu()
    rows = torch.cat([torch.arange(0, 64), torch.arange(Lq - 32, Lq),
                      torch.randperm(Lq, generator=torch.Generator().manual_seed(5))[:64]])
    err, err_exact, _ = _errors(out, q, ids, kp, vp, n_kv, page, rows)
    print(f"max abs err vs quantized-QK oracle {err:.3e}; vs exact attention {err_exact:.3e}")
    assert err <= TOL


def _e4m3_rows(n, heads, seed, pow2):
    g = torch.Generator().manual_seed(seed)
    vals = torch.randint(0, 256, (n, heads, 128), generator=g, dtype=torch.uint8).view(okv.FP8).float()
    vals = torch.where(torch.isnan(vals), torch.zeros_like(vals), vals)
    vals[:, :, 0] = 448.0
    return (vals * 2.0 ** pow2).to(torch.bfloat16)


def test_qk8_equals_exact_kernel_on_representable_rows():
    """Queries and keys that are e4m3 values times powers of two: the quantized-QK scores are the exact ones,
    so the two kernels agree."""
    Lq, H, n_kv, page = 300, 3, 700, 128
    q, ctx, ids, kp, vp = _setup(Lq, H, n_kv, page, 8, seed=70, k=_e4m3_rows(n_kv, H, 71, -8),
                                 q=_e4m3_rows(Lq, H, 72, -9))
    a = attn_paged_fp8(q.to(DEV), ctx, quantized_qk=True).cpu().float()
    b = attn_paged_fp8(q.to(DEV), ctx).cpu().float()
    err = (a - b).abs().max().item()
    print(f"quantized-QK vs exact kernel on representable rows: max abs {err:.3e}")
    assert err <= 2e-3


def test_backend_dispatch_selects_quantized_qk():
    q, ctx, ids, kp, vp = _setup(64, 2, 128, 64, 3, seed=80)
    saved = dict(_WAVE_STATE)
    try:
        enable_hip_fp8_qk()
        assert _WAVE_STATE["attn"] == "hip_fp8_qk"
        got = attend(q.to(DEV).unsqueeze(0), ctx, ctx).cpu()[0]
        want = attn_paged_fp8(q.to(DEV), ctx, quantized_qk=True).cpu()
        assert torch.equal(got, want)
        enable_hip_fp8()
        assert torch.equal(attend(q.to(DEV).unsqueeze(0), ctx, ctx).cpu()[0], attn_paged_fp8(q.to(DEV), ctx).cpu())
    finally:
        _WAVE_STATE.clear()
        _WAVE_STATE.update(saved)
