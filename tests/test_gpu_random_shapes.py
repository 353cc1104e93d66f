"""Seeded random shapes for the KV kernels and the W8A8 GEMM against the CPU oracle.

The pack and the gather-dequant must match bit for bit, and the paged attention must stay within
max |out - oracle| <= 2e-2 (Q, K, V ~ N(0, 1), as in the attention parity tests). The KV shapes are
drawn across the ranges the kernels take:
- token counts that are not a multiple of any block size;
- pages of 16 tokens or more for the pack, 64 or more for attention;
- 1 to 40 heads;
- shuffled page tables over pools with unused pages.
The int8 GEMM must give the oracle's int32 accumulators and bf16 outputs bit for bit over random
M, N (a multiple of 4) and K (a multiple of 16), with and without bias.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oat
from oracle import kv as okv
from oracle import linear as olin
from waveforcing_amd import inputs
from waveforcing_amd.backend import attn_paged_fp8
from waveforcing_amd.fp8 import gemm_i8
from waveforcing_amd.kv import Fp8PagePool, PagedKV

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-2


def _pack_shapes(n, seed):
    rng = np.random.default_rng(seed)
    shapes = []
    for i in range(n):
        T = int(rng.integers(1, 3000))
        H = int(rng.choice([1, 2, 3, 5, 12, 40]))
        page = int(rng.integers(16, 700))
        P = -(-T // page) + int(rng.integers(0, 4))
        shapes.append((T, H, page, P, 1000 * seed + i))
    return shapes


def _attn_shapes(n, seed):
    rng = np.random.default_rng(seed)
    shapes = []
    for i in range(n):
        Lq = int(rng.integers(1, 400))
        n_kv = int(rng.integers(1, 3000))
        H = int(rng.choice([1, 2, 3, 5, 12]))
        page = int(rng.integers(64, 1600))
        P = -(-n_kv // page) + int(rng.integers(0, 3))
        shapes.append((Lq, H, n_kv, page, P, 1000 * seed + i))
    return shapes


@pytest.mark.parametrize("T,H,page,P,seed", _pack_shapes(12, seed=5))
def test_random_pack_unpack_bit_exact(T, H, page, P, seed):
    print(f"pack T={T} H={H} page={page} P={P} seed={seed}", flush=True)
    k = inputs.heavy_tailed_kv(T, H, 128, seed=seed)
    v = inputs.heavy_tailed_kv(T, H, 128, seed=seed + 1)
    ids = inputs.page_table(-(-T // page), P, seed=seed + 2)
    pool = Fp8PagePool(P, H, 128, page, DEV)
    table = pool.page_table(ids)
    pool.pack(k.to(DEV), v.to(DEV), table)
    okc, oks = okv.new_pool(P, page, H, 128)
    ovc, ovs = okv.new_pool(P, page, H, 128)
    okv.pack(k, ids, page, okc, oks)
    okv.pack(v, ids, page, ovc, ovs)
    assert torch.equal(pool.k_codes.cpu(), okc) and torch.equal(pool.k_scales.cpu(), oks)
    assert torch.equal(pool.v_codes.cpu(), ovc) and torch.equal(pool.v_scales.cpu(), ovs)
    ko, vo = pool.unpack(table, T)
    assert torch.equal(ko.cpu(), okv.unpack(ids, T, page, okc, oks))
    assert torch.equal(vo.cpu(), okv.unpack(ids, T, page, ovc, ovs))


@pytest.mark.parametrize("Lq,H,n_kv,page,P,seed", _attn_shapes(12, seed=6))
def test_random_paged_attention(Lq, H, n_kv, page, P, seed):
    print(f"attention Lq={Lq} H={H} n_kv={n_kv} page={page} P={P} seed={seed}", flush=True)
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((n_kv, H, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((n_kv, H, 128), generator=g).to(torch.bfloat16)
    q = torch.randn((Lq, H, 128), generator=g).to(torch.bfloat16)
    ids = inputs.page_table(-(-n_kv // page), P, seed=seed + 3)
    pool = Fp8PagePool(P, H, 128, page, DEV)
    table = pool.page_table(ids)
    pool.pack(k.to(DEV), v.to(DEV), table)
    okc, oks = okv.new_pool(P, page, H, 128)
    ovc, ovs = okv.new_pool(P, page, H, 128)
    okv.pack(k, ids, page, okc, oks)
    okv.pack(v, ids, page, ovc, ovs)
    out = attn_paged_fp8(q.to(DEV), PagedKV(pool, table, n_kv)).cpu()
    ref = oat.paged_fp8(q, (okc, oks), (ovc, ovs), ids, n_kv, page)
    err = (out.float() - ref).abs().max().item()
    print(f"max abs err {err:.3e}")
    assert err <= TOL, err


def _gemm_shapes(n, seed):
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 2500)), 4 * int(rng.integers(1, 1000)), 16 * int(rng.integers(1, 256)),
             bool(rng.integers(0, 2)), 1000 * seed + i) for i in range(n)]


@pytest.mark.parametrize("M,N,K,bias,seed", _gemm_shapes(12, seed=7))
def test_random_gemm_i8_exact(M, N, K, bias, seed):
    print(f"gemm M={M} N={N} K={K} bias={bias} seed={seed}", flush=True)
    x = inputs.outlier_activations(M, K, seed=seed, chan_seed=seed + 1)
    w, b = inputs.linear_weights(N, K, w_seed=seed + 2, b_seed=seed + 3)
    qx, sx = olin.i8_quant_rows(x)
    qw, sw = olin.i8_quant_rows(w)
    acc = torch.empty((M, N), dtype=torch.int32, device=DEV)
    y = gemm_i8(qx.to(DEV), qw.to(DEV), sx.to(DEV), sw.to(DEV), b.to(DEV) if bias else None, acc_out=acc)
    oy, oacc = olin.i8_gemm(qx, qw, sx, sw, b if bias else None)
    assert torch.equal(acc.cpu(), oacc)
    assert torch.equal(y.cpu(), oy)
