"""Run-to-run repeatability of the hot kernels at full size.

Each kernel runs several times on the same inputs. Before every run its outputs are refilled with a
byte pattern that alternates between runs (0x7F, 0x81), and every run must return the first run's
output bit for bit. This catches two faults. An LDS race or a missing wait gives run-dependent
results. An output element the kernel never writes keeps the pattern, so it differs between runs.
The kernels use no atomics and no run-dependent reduction order, so they are deterministic by
construction; this test checks that they are in practice.
"""

import pytest
import torch

from waveforcing_amd import _lib, inputs
from waveforcing_amd.backend import attn_dense_bf16, attn_paged_fp8
from waveforcing_amd.fp8 import gemm_i8
from waveforcing_amd.kv import Fp8PagePool, PagedKV

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
REPS = 8


def _fill(t, i):
    t.view(torch.uint8).fill_(0x7F if i % 2 == 0 else 0x81)


def _normal(shape, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16).to(DEV)


def _assert_repeats(run, outs):
    """``run()`` writes into the tensors of ``outs``; every repetition must equal the first."""
    first = None
    for i in range(REPS):
        for t in outs:
            _fill(t, i)
        run()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs]
        if first is None:
            first = got
        else:
            for a, b in zip(first, got):
                assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), f"run {i} differs"


def test_paged_attention_repeats():
    """1.3B self-attention: 4680 queries x 12 heads over 37440 FP8 paged keys."""
    T, H, D, page, n_kv = 4680, 12, 128, 1560, 37440
    pool = Fp8PagePool(30, H, D, page, DEV)
    table = pool.page_table(inputs.page_table(n_kv // page, 30, seed=3))
    pool.pack(_normal((n_kv, H, D), 1), _normal((n_kv, H, D), 2), table)
    q = _normal((T, H, D), 4)
    out = torch.empty_like(q)
    ctx = PagedKV(pool, table, n_kv)
    _assert_repeats(lambda: attn_paged_fp8(q, ctx, out=out), [out])


@pytest.mark.parametrize("H", [12, 40])
def test_dense_cross_attention_repeats(H):
    """Text cross-attention: 4680 queries over 512 dense bf16 keys."""
    q, k, v = _normal((4680, H, 128), 5), _normal((512, H, 128), 6), _normal((512, H, 128), 7)
    out = torch.empty_like(q)
    _assert_repeats(lambda: attn_dense_bf16(q, k, v, out=out), [out])


@pytest.mark.parametrize("M,N,K", [(4680, 1536, 1536), (4680, 15360, 5120)])
def test_gemm_i8_repeats(M, N, K):
    """The 1.3B linear and the 14B fused QKV: bf16 output and int32 accumulators."""
    g = torch.Generator().manual_seed(M + N + K)
    qx = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(DEV)
    qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(DEV)
    sx = (torch.rand(M, generator=g) * 0.01 + 1e-3).to(DEV)
    sw = (torch.rand(N, generator=g) * 0.01 + 1e-3).to(DEV)
    bias = _normal((N,), 8)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    acc = torch.empty((M, N), dtype=torch.int32, device=DEV)
    _assert_repeats(lambda: gemm_i8(qx, qw, sx, sw, bias, acc_out=acc, out=y), [y, acc])


def test_act_quant_repeats():
    """Per-token int8 quantization of an FFN-wide activation (4680 x 8960)."""
    x = inputs.outlier_activations(4680, 8960, seed=9, chan_seed=10).to(DEV)
    q = torch.empty((4680, 8960), dtype=torch.int8, device=DEV)
    s = torch.empty((4680,), dtype=torch.float32, device=DEV)
    st = _lib.stream_handle(DEV)
    _assert_repeats(lambda: _lib.call("wf_act_quant_i8", x.data_ptr(), 4680, 8960, 8960, q.data_ptr(), s.data_ptr(),
                                      st), [q, s])


def test_kv_pack_repeats():
    """One 1.3B chunk's K/V pack (4680 tokens = 3 whole pages, so every element of the used pages is
    written); only the used pages are compared, the others keep the fill pattern."""
    T, H, D, page, P = 4680, 12, 128, 1560, 6
    ids = inputs.page_table(3, P, seed=11)
    pool = Fp8PagePool(P, H, D, page, DEV)
    table = pool.page_table(ids)
    k = inputs.heavy_tailed_kv(T, H, D, seed=12).to(DEV)
    v = inputs.heavy_tailed_kv(T, H, D, seed=13).to(DEV)
    first = None
    for i in range(REPS):
        for t in (pool.k_codes, pool.k_scales, pool.v_codes, pool.v_scales):
            _fill(t, i)
        pool.pack(k, v, table)
        torch.cuda.synchronize()
        got = [t[ids].clone() for t in (pool.k_codes, pool.k_scales, pool.v_codes, pool.v_scales)]
        if first is None:
            first = got
        else:
            for a, b in zip(first, got):
                assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), f"run {i} differs"
