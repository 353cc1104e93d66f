"""GPU parity of the fused K/V producers that feed the FP8 pages.

* ``wf_fp8_kv_pack_rope`` (anchor re-RoPE + pack): codes and scales equal,
  bit for bit, the oracle's pack of the oracle's table rotation
  (oracle.block.rope_apply_table, pinned on the CPU) of the same K; V equals
  the oracle's plain pack.
* ``wf_k_norm_rope_kv_pack`` (K RMSNorm + RoPE + K/V pack from the QKV
  output): bit-exact against the unfused chain wf_rmsnorm_rope ->
  wf_fp8_kv_pack on the same device; its un-rotated output equals
  wf_rmsnorm_rope without tables; the oracle's rotation + pack of that output
  gives the same codes; the normalized K is within bf16 rounding of the
  oracle's RMSNorm.
Shapes cover the 1.3B and 14B head counts, partial pages, a 16384-wide row
(128 heads, one workgroup per row), tokens whose logical page is invalid,
in-place un-rotated output and argument errors.
"""

import pytest
import torch

from oracle import block as ob
from oracle import kv as okv
from waveforcing_amd import _lib, inputs, rope
from waveforcing_amd.kv import Fp8PagePool, PageTable

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
EPS = 1e-6


def _grid_for(T):
    # a (frames, height, width) grid of exactly T tokens
    for f in (3, 2, 1):
        if T % f == 0:
            hw = T // f
            for h in range(int(hw ** 0.5), 0, -1):
                if hw % h == 0:
                    return f, h, hw // h
    return 1, 1, T


def _tables(T, start_frame):
    f, h, w = _grid_for(T)
    return rope.cos_sin(f, h, w, start_frame, 128, device=DEV)


def _pools_cpu(pool):
    return pool.k_codes.cpu(), pool.k_scales.cpu(), pool.v_codes.cpu(), pool.v_scales.cpu()


@pytest.mark.parametrize("T,H,page,P,start,seed", [
    (4680, 12, 1560, 6, 9, 0),     # one 1.3B chunk re-RoPEd to frame 9
    (4680, 40, 1560, 4, 3, 1),     # 14B heads
    (1000, 12, 1560, 2, 0, 2),     # partial page, frame 0
    (257, 3, 16, 20, 21, 3),       # small pages
])
def test_pack_rope_matches_oracle(T, H, page, P, start, seed):
    k = inputs.heavy_tailed_kv(T, H, 128, seed=3000 + seed)
    v = inputs.heavy_tailed_kv(T, H, 128, seed=4000 + seed)
    cos, sin = _tables(T, start)
    ids = inputs.page_table(-(-T // page), P, seed=seed)
    pool = Fp8PagePool(P, H, 128, page, DEV)
    pool.pack(k.to(DEV), v.to(DEV), pool.page_table(ids), rope=(cos, sin))
    kc, ks, vc, vs = _pools_cpu(pool)
    okc, oks = okv.new_pool(P, page, H, 128)
    ovc, ovs = okv.new_pool(P, page, H, 128)
    okv.pack(ob.rope_apply_table(k, cos.cpu(), sin.cpu()), ids, page, okc, oks)
    okv.pack(v, ids, page, ovc, ovs)
    assert torch.equal(kc, okc) and torch.equal(ks, oks)
    assert torch.equal(vc, ovc) and torch.equal(vs, ovs)


def test_pack_rope_identity_table_equals_plain_pack():
    k = inputs.heavy_tailed_kv(300, 4, 128, seed=11)
    one = torch.ones((300, 64), dtype=torch.float32, device=DEV)
    zero = torch.zeros((300, 64), dtype=torch.float32, device=DEV)
    a = Fp8PagePool(3, 4, 128, 128, DEV)
    b = Fp8PagePool(3, 4, 128, 128, DEV)
    a.pack(k.to(DEV), None, a.page_table([2, 0, 1]), rope=(one, zero))
    b.pack(k.to(DEV), None, b.page_table([2, 0, 1]))
    assert torch.equal(a.k_codes, b.k_codes) and torch.equal(a.k_scales, b.k_scales)


def _qkv(T, dim, seed):
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn((T, 3 * dim), generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn((dim,), generator=g)).to(torch.bfloat16)
    return qkv, w


@pytest.mark.parametrize("T,H,page,P,start,seed", [
    (4680, 12, 1560, 6, 6, 0),     # 1.3B chunk (one wave per row, 3 chunks per lane)
    (4680, 40, 1560, 4, 3, 1),     # 14B chunk (one workgroup per row)
    (1001, 16, 256, 9, 0, 2),      # 2048-wide rows, 4 chunks per lane, partial page
    (40, 128, 16, 4, 5, 3),        # 16384-wide rows, 8 chunks per lane
])
def test_k_norm_rope_pack_equals_unfused_chain(T, H, page, P, start, seed):
    dim = H * 128
    qkv, w = _qkv(T, dim, seed)
    cos, sin = _tables(T, start)
    ids = inputs.page_table(-(-T // page), P, seed=seed)
    d = qkv.to(DEV)
    wd = w.to(DEV)
    k, v = d[:, dim:2 * dim], d[:, 2 * dim:]

    fused = Fp8PagePool(P, H, 128, page, DEV)
    table = fused.page_table(ids)
    ku = torch.empty((T, dim), dtype=torch.bfloat16, device=DEV)
    fused.pack_k_norm_rope(k, v, table, wd, EPS, (cos, sin), ku_out=ku)

    ref = Fp8PagePool(P, H, 128, page, DEV)
    kr = torch.empty((T, dim), dtype=torch.bfloat16, device=DEV)
    kn = torch.empty((T, dim), dtype=torch.bfloat16, device=DEV)
    for out, tabs in ((kr, (cos, sin)), (kn, (None, None))):
        _lib.call("wf_rmsnorm_rope", k.data_ptr(), T, dim, k.stride(0), 128, EPS, wd.data_ptr(), _lib.ptr(tabs[0]),
                  _lib.ptr(tabs[1]), out.data_ptr(), out.stride(0), _lib.stream_handle(DEV))
    ref.pack(kr.view(T, H, 128), v.reshape(T, H, 128), ref.page_table(ids))
    for a, b in zip(_pools_cpu(fused), _pools_cpu(ref)):
        assert torch.equal(a, b)
    assert torch.equal(ku, kn)

    # oracle: the table rotation + pack of the un-rotated output gives the same codes,
    # and that output is the RMSNorm to within bf16 rounding
    kc, ks, _, _ = _pools_cpu(fused)
    okc, oks = okv.new_pool(P, page, H, 128)
    okv.pack(ob.rope_apply_table(ku.cpu().view(T, H, 128), cos.cpu(), sin.cpu()), ids, page, okc, oks)
    assert torch.equal(kc, okc) and torch.equal(ks, oks)
    want = ob.rms_norm(qkv[:, dim:2 * dim], w).float()
    got = ku.cpu().float()
    assert bool(((got - want).abs() <= want.abs() * 2 ** -6 + 1e-6).all())
    assert float((got != want).double().mean()) < 0.01


def test_k_norm_pack_without_rope_or_v_and_in_place():
    T, H, page, P = 500, 12, 128, 5
    dim = H * 128
    qkv, w = _qkv(T, dim, 21)
    d = qkv.to(DEV)
    wd = w.to(DEV)
    k = d[:, dim:2 * dim]
    ids = [4, 0, 3, 1]
    a = Fp8PagePool(P, H, 128, page, DEV)
    kn = torch.empty((T, dim), dtype=torch.bfloat16, device=DEV)
    _lib.call("wf_rmsnorm_rope", k.data_ptr(), T, dim, k.stride(0), 128, EPS, wd.data_ptr(), None, None,
              kn.data_ptr(), kn.stride(0), _lib.stream_handle(DEV))
    a.pack_k_norm_rope(k, None, a.page_table(ids), wd, EPS, None, ku_out=k)   # in place, K only
    assert torch.equal(k, kn)
    assert int(a.v_codes.abs().sum()) == 0
    okc, oks = okv.new_pool(P, page, H, 128)
    okv.pack(kn.cpu().view(T, H, 128), ids, page, okc, oks)
    assert torch.equal(a.k_codes.cpu(), okc) and torch.equal(a.k_scales.cpu(), oks)


def test_k_norm_pack_skips_invalid_pages():
    T, H, page, P = 48, 2, 16, 3
    dim = H * 128
    qkv, w = _qkv(T, dim, 31)
    d = qkv.to(DEV)
    k, v = d[:, dim:2 * dim], d[:, 2 * dim:]
    pool = Fp8PagePool(P, H, 128, page, DEV)
    table = PageTable([0, 1, 2], P, DEV)
    table.dev = torch.tensor([1, 7, -1], dtype=torch.int32, device=DEV)  # bypass host validation
    ku = torch.empty((T, dim), dtype=torch.bfloat16, device=DEV)
    pool.pack_k_norm_rope(k, v, table, w.to(DEV), EPS, None, ku_out=ku)
    okc, oks = okv.new_pool(P, page, H, 128)
    ovc, ovs = okv.new_pool(P, page, H, 128)
    okv.pack(ku.cpu().view(T, H, 128), [1, 7, -1], page, okc, oks)
    okv.pack(qkv[:, 2 * dim:].reshape(T, H, 128), [1, 7, -1], page, ovc, ovs)
    assert torch.equal(pool.k_codes.cpu(), okc) and torch.equal(pool.k_scales.cpu(), oks)
    assert torch.equal(pool.v_codes.cpu(), ovc) and torch.equal(pool.v_scales.cpu(), ovs)
    assert int(pool.k_codes[0].abs().sum()) == 0 and int(pool.k_codes[2].abs().sum()) == 0


def test_fused_pack_argument_errors():
    pool = Fp8PagePool(2, 2, 128, 16, DEV)
    table = pool.page_table([0, 1])
    k = torch.zeros((20, 256), dtype=torch.bfloat16, device=DEV)
    w = torch.ones((256,), dtype=torch.bfloat16, device=DEV)
    cos = torch.ones((20, 64), dtype=torch.float32, device=DEV)
    with pytest.raises(RuntimeError, match="both be given"):
        _lib.call("wf_k_norm_rope_kv_pack", k.data_ptr(), None, 20, 2, 128, 256, EPS, w.data_ptr(), cos.data_ptr(),
                  None, None, 0, table.dev.data_ptr(), 2, 16, pool.k_codes.data_ptr(), None,
                  pool.k_scales.data_ptr(), None, 2, _lib.stream_handle(DEV))
    with pytest.raises(RuntimeError, match="exceeds 16384"):
        _lib.call("wf_k_norm_rope_kv_pack", k.data_ptr(), None, 1, 130, 128, 130 * 128, EPS, w.data_ptr(), None,
                  None, None, 0, table.dev.data_ptr(), 2, 16, pool.k_codes.data_ptr(), None,
                  pool.k_scales.data_ptr(), None, 2, _lib.stream_handle(DEV))
    with pytest.raises(RuntimeError, match="not overlap"):
        _lib.call("wf_k_norm_rope_kv_pack", k.data_ptr(), None, 20, 2, 128, 256, EPS, w.data_ptr(), None, None,
                  k.data_ptr() + 256, 256, table.dev.data_ptr(), 2, 16, pool.k_codes.data_ptr(), None,
                  pool.k_scales.data_ptr(), None, 2, _lib.stream_handle(DEV))
    with pytest.raises(RuntimeError, match="null RoPE table"):
        _lib.call("wf_fp8_kv_pack_rope", k.data_ptr(), None, 20, 2, 128, 256, None, None, table.dev.data_ptr(), 2,
                  16, pool.k_codes.data_ptr(), None, pool.k_scales.data_ptr(), None, 2, _lib.stream_handle(DEV))
    with pytest.raises(ValueError, match="rope cos"):
        pool.pack(k.view(20, 2, 128), None, table, rope=(cos[:10], cos[:10]))
    torch.cuda.synchronize()


@pytest.mark.parametrize("T,H,page,P,start,seed", [
    (4680, 12, 1560, 6, 6, 0),     # 1.3B (one wave per row)
    (4680, 40, 1560, 4, 3, 1),     # 14B (one workgroup per row: the q reduction has its own LDS slots)
    (40, 128, 16, 4, 5, 3),        # 16384-wide rows
])
def test_qk_norm_rope_pack_equals_separate_q_pass(T, H, page, P, start, seed):
    dim = H * 128
    qkv, w = _qkv(T, dim, seed)
    wq = (1 + 0.1 * torch.randn((dim,), generator=torch.Generator().manual_seed(seed + 50))).to(torch.bfloat16)
    cos, sin = _tables(T, start)
    ids = inputs.page_table(-(-T // page), P, seed=seed)
    a = qkv.to(DEV)
    b = qkv.to(DEV)
    wd, wqd = w.to(DEV), wq.to(DEV)
    ku_a = torch.empty((T, dim), dtype=torch.bfloat16, device=DEV)
    ku_b = torch.empty_like(ku_a)
    fused = Fp8PagePool(P, H, 128, page, DEV)
    fused.pack_k_norm_rope(a[:, dim:2 * dim], a[:, 2 * dim:], fused.page_table(ids), wd, EPS, (cos, sin), ku_out=ku_a,
                           q=a[:, :dim], norm_q=wqd)
    ref = Fp8PagePool(P, H, 128, page, DEV)
    qb = b[:, :dim]
    _lib.call("wf_rmsnorm_rope", qb.data_ptr(), T, dim, qb.stride(0), 128, EPS, wqd.data_ptr(), cos.data_ptr(),
              sin.data_ptr(), qb.data_ptr(), qb.stride(0), _lib.stream_handle(DEV))
    ref.pack_k_norm_rope(b[:, dim:2 * dim], b[:, 2 * dim:], ref.page_table(ids), wd, EPS, (cos, sin), ku_out=ku_b)
    assert torch.equal(a, b)                         # q rewritten identically, K and V untouched
    assert torch.equal(ku_a, ku_b)
    for x, y in zip(_pools_cpu(fused), _pools_cpu(ref)):
        assert torch.equal(x, y)


def test_qk_norm_rope_pack_rejects_overlapping_q():
    T, H, page = 8, 2, 16
    dim = H * 128
    d = torch.zeros((T, 3 * dim), dtype=torch.bfloat16, device=DEV)
    w = torch.ones((dim,), dtype=torch.bfloat16, device=DEV)
    pool = Fp8PagePool(2, H, 128, page, DEV)
    table = pool.page_table([0])
    k = d[:, dim:2 * dim]
    with pytest.raises(RuntimeError, match="must not overlap"):
        pool.pack_k_norm_rope(k, None, table, w, EPS, None, q=d[:, dim - 64:2 * dim - 64], norm_q=w)
    with pytest.raises(ValueError, match="norm_q"):
        pool.pack_k_norm_rope(k, None, table, w, EPS, None, q=d[:, :dim])
    torch.cuda.synchronize()
