"""Pins the attention oracle (oracle/attention.py) on the CPU.

Closed forms: constant V returns V; a single key returns its V row;
identical keys give the mean of V; a zero scale gives the mean of V; key
order does not matter; and a float64 numpy evaluation of the definition
agrees on random data.  The paged path equals attention over the plain
concatenation of the dequantized rows (paging changes layout only).
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
