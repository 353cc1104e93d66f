"""GPU parity of the paged FP8 attention against the CPU oracle.

Bar (the attention workload: Q, K, V ~ N(0, 1)): max |out - oracle| <= 2e-2
for the bf16 output; the oracle attends in fp32 over the bf16-dequantized
pages, the kernel over code * scale exactly.  With heavy-tailed K/V (the KV
workload's Student-t(3) outliers) outputs reach magnitudes where one bf16
ulp alone exceeds 2e-2, so that case is held to 2e-2 * max(1, |oracle|).
Full-size cases (37440 keys) compare a sample of query rows, all heads.
"""

import math

import pytest
import torch

from oracle import attention as oat
from oracle import kv as okv
from waveforcing_amd import _lib, inputs
from waveforcing_amd.backend import _WAVE_STATE, attend, attn_dense_bf16, attn_paged_fp8, enable_hip_fp8
from waveforcing_amd.kv import Fp8PagePool, PagedKV

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-2


def _normal(shape, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)


def _setup(Lq, H, n_kv, page, P, seed, const_v=False, heavy=False):
    if heavy:
        k = inputs.heavy_tailed_kv(n_kv, H, 128, seed=seed)
        v = inputs.heavy_tailed_kv(n_kv, H, 128, seed=seed + 1)
    else:
        k = _normal((n_kv, H, 128), seed)
        v = _normal((n_kv, H, 128), seed + 1)
    if const_v:
        v = v[:1].expand(n_kv, H, 128).contiguous()
    g = torch.Generator().manual_seed(seed + 2)
    q = torch.randn((Lq, H, 128), generator=g).to(torch.bfloat16)
    n_pages = -(-n_kv // page)
    ids = inputs.page_table(n_pages, P, seed=seed + 3)
    pool = Fp8PagePool(P, H, 128, page, DEV)
    table = pool.page_table(ids)
    pool.pack(k.to(DEV), v.to(DEV), table)
    okc, oks = okv.new_pool(P, page, H, 128)
    ovc, ovs = okv.new_pool(P, page, H, 128)
    okv.pack(k, ids, page, okc, oks)
    okv.pack(v, ids, page, ovc, ovs)
    return q, pool, PagedKV(pool, table, n_kv), ids, (okc, oks), (ovc, ovs), v


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
def test_paged_attention_matches_oracle(Lq, H, n_kv, page, P, seed):
    q, pool, ctx, ids, kp, vp, _ = _setup(Lq, H, n_kv, page, P, seed)
    out = attn_paged_fp8(q.to(DEV).unsqueeze(0), ctx).cpu()[0]
    ref = oat.paged_fp8(q, kp, vp, ids, n_kv, page)
    err = (out.float() - ref).abs().max().item()
    print(f"max abs err {err:.3e}")
    assert err <= TOL, err


def test_heavy_tailed_relative():
    Lq, H, n_kv, page = 128, 12, 4680, 1560
    q, pool, ctx, ids, kp, vp, _ = _setup(Lq, H, n_kv, page, 6, seed=40, heavy=True)
    out = attn_paged_fp8(q.to(DEV), ctx).cpu().float()
    ref = oat.paged_fp8(q, kp, vp, ids, n_kv, page)
    rel = ((out - ref).abs() / ref.abs().clamp(min=1.0)).max().item()
    print(f"max rel err {rel:.3e}, max abs err {(out - ref).abs().max().item():.3e}")
    assert rel <= TOL, rel


def test_full_context_sampled_rows():
    """Lq 4680 queries over 8 chunks (37440 keys), 12 heads; 160 sampled rows."""
    Lq, H, n_kv, page = 4680, 12, 37440, 1560
    P = 30
    q, pool, ctx, ids, kp, vp, _ = _setup(Lq, H, n_kv, page, P, seed=10)
    out = attn_paged_fp8(q.to(DEV), ctx).cpu()
    rows = torch.cat([torch.arange(0, 64), torch.arange(Lq - 32, Lq),
                      torch.randperm(Lq, generator=torch.Generator().manual_seed(5))[:64]])
    ref = oat.paged_fp8(q[rows], kp, vp, ids, n_kv, page)
    err = (out[rows].float() - ref).abs().max().item()
    print(f"max abs err {err:.3e}")
    assert err <= TOL, err


def test_full_context_14b_heads_sampled_rows():
    """The 14B geometry: 4680 queries x 40 heads over 8 chunks (37440 keys); 160 sampled rows, all heads."""
    Lq, H, n_kv, page = 4680, 40, 37440, 1560
    q, pool, ctx, ids, kp, vp, _ = _setup(Lq, H, n_kv, page, 26, seed=50)
    out = attn_paged_fp8(q.to(DEV), ctx).cpu()
    rows = torch.cat([torch.arange(0, 64), torch.arange(Lq - 32, Lq),
                      torch.randperm(Lq, generator=torch.Generator().manual_seed(6))[:64]])
    ref = oat.paged_fp8(q[rows], kp, vp, ids, n_kv, page)
    err = (out[rows].float() - ref).abs().max().item()
    print(f"max abs err {err:.3e}")
    assert err <= TOL, err


@pytest.mark.parametrize("H", [12, 40])
def test_dense_cross_attention_full_size(H):
    """The text cross-attention: 4680 queries over 512 dense bf16 text keys (wf_attn_dense_bf16), all rows."""
    g = torch.Generator().manual_seed(60 + H)
    q = torch.randn((4680, H, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((512, H, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((512, H, 128), generator=g).to(torch.bfloat16)
    out = attn_dense_bf16(q.to(DEV), k.to(DEV), v.to(DEV)).cpu().float()
    ref = oat.sdpa(q, k, v)
    err = (out - ref).abs().max().item()
    print(f"H={H}: max abs err {err:.3e}")
    assert err <= TOL, err


def test_constant_v_returns_v():
    q, pool, ctx, ids, kp, vp, v = _setup(200, 2, 500, 128, 5, seed=20, const_v=True)
    out = attn_paged_fp8(q.to(DEV), ctx).cpu().float()
    cv, sv = okv.quantize_rows(v[:1])
    vrow = okv.dequantize_rows(cv, sv).float()
    assert (out - vrow.expand_as(out)).abs().max().item() <= 1e-2


def test_single_key_returns_its_value_exactly():
    """One key: its weight is 2^0 rounded to bf16 (1.0) and the row sum 1, the masked keys weigh 0, so
    every query's output row is that key's dequantized V, bf16(code * scale), bit for bit."""
    q, pool, ctx, ids, kp, vp, v = _setup(70, 3, 1, 64, 2, seed=40)
    out = attn_paged_fp8(q.to(DEV), ctx).cpu()
    cv, sv = okv.quantize_rows(v[:1])
    vrow = okv.dequantize_rows(cv, sv)
    assert torch.equal(out, vrow.expand_as(out))


@pytest.mark.parametrize("entry", ["wf_attn_paged_fp8", "wf_attn_paged_fp8_qk8"])
def test_invalid_page_ids_read_as_zero_keys(entry):
    """Table entries outside the pool (-1, or the pool size) read as zero codes and zero scales: their keys
    score 0 and carry V = 0.  Pages of 200 tokens hold several tiles and tiles straddle page ends, so the
    kernel moves its page bases within valid and invalid pages and recomputes them at every page start.
    Such tables reach the kernel only through the C ABI (the Python page table refuses them)."""
    Lq, H, page, P = 96, 3, 200, 6
    n_kv = 4 * page + 77
    k, v, q = _normal((n_kv, H, 128), 70), _normal((n_kv, H, 128), 71), _normal((Lq, H, 128), 72)
    ids = [4, 0, 5, 2, 1]
    pool = Fp8PagePool(P, H, 128, page, DEV)
    pool.pack(k.to(DEV), v.to(DEV), pool.page_table(ids))
    bad = list(ids)
    bad[1], bad[3] = -1, P
    table = torch.tensor(bad, dtype=torch.int32, device=DEV)
    qd = q.to(DEV)
    out = torch.empty((Lq, H, 128), dtype=torch.bfloat16, device=DEV)
    _lib.call(entry, qd.data_ptr(), Lq, H, 128, qd.stride(0), pool.k_codes.data_ptr(), pool.v_codes.data_ptr(),
              pool.k_scales.data_ptr(), pool.v_scales.data_ptr(), P, page, table.data_ptr(), len(bad), n_kv,
              1.0 / math.sqrt(128), out.data_ptr(), out.stride(0), _lib.stream_handle(DEV))
    kc, ks = okv.quantize_rows(k)
    vz = okv.dequantize_rows(*okv.quantize_rows(v)).clone()
    for lp in (1, 3):
        rows = slice(lp * page, (lp + 1) * page)
        kc[rows], ks[rows], vz[rows] = 0, 0.0, 0
    kz = okv.dequantize_rows(kc, ks)
    ref = oat.sdpa(q, kz, vz) if entry == "wf_attn_paged_fp8" else oat.sdpa_qk8(q, kc, ks, vz)
    err = (out.cpu().float() - ref).abs().max().item()
    print(f"{entry}: max abs err {err:.3e}")
    assert err <= TOL, err


def test_backend_dispatch_and_scale():
    q, pool, ctx, ids, kp, vp, _ = _setup(64, 2, 300, 128, 4, seed=30)
    saved = dict(_WAVE_STATE)
    try:
        enable_hip_fp8()
        out = attend(q.to(DEV).unsqueeze(0), ctx, ctx)
        assert out.shape == (1, 64, 2, 128)
        ref = oat.paged_fp8(q, kp, vp, ids, 300, 128)
        assert (out[0].cpu().float() - ref).abs().max().item() <= TOL
        half = attn_paged_fp8(q.to(DEV), ctx, softmax_scale=0.5 / math.sqrt(128)).cpu()
        ref2 = oat.paged_fp8(q, kp, vp, ids, 300, 128, scale=0.5 / math.sqrt(128))
        assert (half.float() - ref2).abs().max().item() <= TOL
        with pytest.raises(ValueError):
            attn_paged_fp8(q.to(DEV), ctx, causal=True)
    finally:
        _WAVE_STATE.clear()
        _WAVE_STATE.update(saved)


def test_empty_context_writes_zeros():
    """n_kv = 0: an empty softmax gives every query zero weight, so the output rows are zeros (no pools are
    read; null pool pointers are accepted)."""
    H, Lq = 2, 70
    q = _normal((Lq, H, 128), 70).to(DEV)
    out = torch.full((Lq, H, 128), 7.0, dtype=torch.bfloat16, device=DEV)
    _lib.call("wf_attn_paged_fp8", q.data_ptr(), Lq, H, 128, H * 128, None, None, None, None, 0, 64, None, 0, 0,
              128 ** -0.5, out.data_ptr(), H * 128, _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0


def test_page_ids_outside_the_pool_read_as_zero_keys():
    """A page-table entry outside [0, pool_pages) is never read: its keys enter the softmax with K = 0
    (score 0) and V = 0, as include/wf_api.h states.  Raw C call (the Python PageTable refuses such ids)."""
    H, Lq, page, n_kv, P = 2, 100, 64, 3 * 64 - 10, 5
    q, pool, ctx, ids, kp, vp, _ = _setup(Lq, H, n_kv, page, P, seed=80)
    table = torch.tensor([ids[0], -1, P + 3], dtype=torch.int32, device=DEV)
    out = torch.empty((Lq, H, 128), dtype=torch.bfloat16, device=DEV)
    qd = q.to(DEV)
    _lib.call("wf_attn_paged_fp8", qd.data_ptr(), Lq, H, 128, H * 128, pool.k_codes.data_ptr(),
              pool.v_codes.data_ptr(), pool.k_scales.data_ptr(), pool.v_scales.data_ptr(), P, page,
              table.data_ptr(), 3, n_kv, 128 ** -0.5, out.data_ptr(), H * 128, _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    k = okv.unpack(ids, n_kv, page, *kp)
    v = okv.unpack(ids, n_kv, page, *vp)
    k[page:] = 0
    v[page:] = 0
    ref = oat.sdpa(q, k, v)
    err = (out.cpu().float() - ref).abs().max().item()
    print(f"max abs err {err:.3e}")
    assert err <= TOL, err
    # and the zero keys do weigh in: attending to the valid page alone differs
    alone = oat.sdpa(q, k[:page], v[:page])
    assert (alone - ref).abs().max().item() > 10 * TOL
