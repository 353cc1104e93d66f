"""GPU parity of the int8 W8A8 path against the CPU oracle.

Bars: int8 codes and fp32 scales bit-exact; int32 accumulators exact; bf16
outputs bit-exact for the plain epilogue (same fp32 operation order), and
within 1e-2 relative error (the stated tolerance) with the GELU-tanh
epilogue, whose tanh differs between the GPU and CPU math libraries.
"""

import pytest
import torch

from oracle import linear as olin
from waveforcing_amd import inputs
from waveforcing_amd.fp8 import WaveW8A8Linear, _quant_rows_i8, gemm_i8, quantize_transformer_w8a8

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("M,K,seed", [(4680, 1536, 0), (1, 16, 1), (37, 48, 2), (300, 8960, 3), (5, 4112, 4),
                                      (4680, 5120, 5)])
def test_quant_rows_bit_exact(M, K, seed):
    x = inputs.outlier_activations(M, K, seed=seed, chan_seed=seed + 10)
    q, s = _quant_rows_i8(x.to(DEV))
    oq, os_ = olin.i8_quant_rows(x)
    assert torch.equal(s.cpu(), os_)
    assert torch.equal(q.cpu(), oq)


def test_quant_rows_exact_ties_and_zero_rows():
    e = torch.tensor([-3.0, 0.0, 2.0, 5.0])
    k = torch.arange(-64, 64, dtype=torch.float32)
    rows = torch.cat([torch.full((4, 1), 127.0), (k[None, :] + 0.5).expand(4, -1), torch.zeros(4, 15)], 1)
    rows = (rows * torch.pow(2.0, e)[:, None]).to(torch.bfloat16)
    rows = torch.cat([rows, torch.zeros((2, rows.shape[1]), dtype=torch.bfloat16)])
    q, s = _quant_rows_i8(rows.to(DEV))
    oq, os_ = olin.i8_quant_rows(rows)
    assert torch.equal(s.cpu(), os_) and torch.equal(q.cpu(), oq)


def test_quant_rows_random_scale_ties():
    """Quotients that land on k + 1/2 after fp32 rounding (non-power-of-two scales)."""
    g = torch.Generator().manual_seed(9)
    x = (torch.randint(-254, 255, (2048, 256), generator=g).float() / 2).to(torch.bfloat16)
    x[:, 0] = torch.linspace(1, 120, 2048).to(torch.bfloat16)
    q, s = _quant_rows_i8(x.to(DEV))
    oq, os_ = olin.i8_quant_rows(x)
    assert torch.equal(s.cpu(), os_) and torch.equal(q.cpu(), oq)


def _gemm_case(M, N, K, seed, bias=True, gelu=False):
    x = inputs.outlier_activations(M, K, seed=seed, chan_seed=seed + 1)
    w, b = inputs.linear_weights(N, K, w_seed=seed + 2, b_seed=seed + 3)
    qx, sx = olin.i8_quant_rows(x)
    qw, sw = olin.i8_quant_rows(w)
    acc = torch.empty((M, N), dtype=torch.int32, device=DEV)
    y = gemm_i8(qx.to(DEV), qw.to(DEV), sx.to(DEV), sw.to(DEV), b.to(DEV) if bias else None, gelu=gelu,
                acc_out=acc)
    oy, oacc = olin.i8_gemm(qx, qw, sx, sw, b if bias else None, gelu=gelu)
    return y.cpu(), acc.cpu(), oy, oacc


@pytest.mark.parametrize("M,N,K", [
    (4680, 1536, 1536),   # single 1.3B linear
    (4680, 4608, 1536),   # fused QKV
    (4680, 1536, 8960),   # fc_out
    (1, 4, 16), (17, 132, 48), (300, 256, 1552), (513, 1540, 272),
    (3000, 3204, 272),    # more tiles than CUs (several rounds), partial tiles, N % 8 == 4: 8-byte stores
    (2050, 8196, 160),    # 561 tiles, K tail of 32 bytes
    # shapes that take the 256 x 256 workgroup tile (two LDS stages): the 1.3B fc_in, its M / N / K tails
    # (72 rows in the last tile row, a 252-column last tile with N % 8 == 4, a 16-byte K tail), and K loops
    # of one and two steps
    (4680, 8960, 1536), (4680, 8956, 1552), (4680, 8960, 16), (4680, 8960, 144),
])
def test_gemm_exact(M, N, K):
    y, acc, oy, oacc = _gemm_case(M, N, K, seed=M + N + K)
    assert torch.equal(acc, oacc)
    assert torch.equal(y, oy)


@pytest.mark.parametrize("N,K,gelu", [
    (15360, 5120, False),   # 14B fused QKV
    (5120, 5120, False),    # 14B O
    (13824, 5120, True),    # 14B fc_in + GELU
    (5120, 13824, False),   # 14B fc_out
])
def test_gemm_14b_shapes_sampled_rows(N, K, gelu):
    """The 14B block's linears on a 4680-token chunk; int32 accumulators exact and bf16 outputs exact (GELU:
    within the stated tolerance) on 288 rows: the first two and the last tile rows, and random rows."""
    M = 4680
    seed = N + K
    x = inputs.outlier_activations(M, K, seed=seed, chan_seed=seed + 1)
    w, b = inputs.linear_weights(N, K, w_seed=seed + 2, b_seed=seed + 3)
    qx, sx = olin.i8_quant_rows(x)
    qw, sw = olin.i8_quant_rows(w)
    del x, w
    acc = torch.empty((M, N), dtype=torch.int32, device=DEV)
    y = gemm_i8(qx.to(DEV), qw.to(DEV), sx.to(DEV), sw.to(DEV), b.to(DEV), gelu=gelu, acc_out=acc).cpu()
    rows = torch.cat([torch.arange(0, 256, 8), torch.arange(M - 128, M),
                      torch.randperm(M, generator=torch.Generator().manual_seed(seed))[:128]])
    acc = acc.cpu()[rows]
    oy, oacc = olin.i8_gemm(qx[rows].contiguous(), qw, sx[rows].contiguous(), sw, b, gelu=gelu)
    assert torch.equal(acc, oacc)
    if gelu:
        rel = (y[rows].float() - oy.float()).norm() / oy.float().norm()
        assert rel < 1e-2, float(rel)
    else:
        assert torch.equal(y[rows], oy)


@pytest.mark.parametrize("M,N,K", [
    (4680, 5120, 4096),    # one round and a partly covered tile row (the 14B O / fc_out plan)
    (4680, 5112, 4112),    # the same plan with a 248-column last tile and a 16-byte K tail
    (4680, 15360, 4096),   # four rounds, then the rest (the 14B QKV plan)
    (4680, 13824, 4096),   # three rounds, then the rest (the 14B fc_in plan)
])
def test_gemm_tile_plans_exact(M, N, K):
    """Shapes planned (on 256 CUs) as whole rounds of 256 x 256 tiles followed by a launch of 128 x 256 tiles
    over the rest: every element of the int32 accumulators equals torch._int_mm (exact integer products), and
    every bf16 output equals the epilogue (float(acc) * sx) * sw + bias evaluated by torch in that order, so a
    tile that no launch covers, or covers twice with different rows, fails.  Outputs start as a fill pattern."""
    g = torch.Generator(device=DEV).manual_seed(M + N + K)
    qx = torch.randint(-127, 128, (M, K), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    qw = torch.randint(-127, 128, (N, K), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    sx = torch.rand((M,), generator=g, device=DEV) * 1e-3
    sw = torch.rand((N,), generator=g, device=DEV) * 1e-3
    b = torch.randn((N,), generator=g, device=DEV).to(torch.bfloat16)
    acc = torch.full((M, N), 0x7f7f7f7f, dtype=torch.int32, device=DEV)
    y = torch.full((M, N), 7.0, dtype=torch.bfloat16, device=DEV)
    gemm_i8(qx, qw, sx, sw, b, acc_out=acc, out=y)
    ref = torch._int_mm(qx, qw.t())
    assert torch.equal(acc, ref)
    yr = ((ref.float() * sx[:, None]) * sw[None, :] + b.float()[None, :]).to(torch.bfloat16)
    assert torch.equal(y, yr)


@pytest.mark.parametrize("seed", range(8))
def test_gemm_random_large_shapes_exact(seed):
    """Seeded large shapes (M 1500-9000, N 3200-17600 in steps of 8, K 4096-6384 in steps of 16) that the
    planner splits in several ways (the 256-row tile over the whole output, or whole rounds of it followed by
    128-row tiles over rectangles with ragged row and column ends): int32 accumulators equal torch._int_mm
    and bf16 outputs equal the torch-evaluated epilogue, element for element."""
    import random

    r = random.Random(seed)
    M, N, K = r.randrange(1500, 9000), 8 * r.randrange(400, 2200), 16 * r.randrange(256, 400)
    print(f"seed {seed}: {M} x {N} x {K}")
    g = torch.Generator(device=DEV).manual_seed(seed)
    qx = torch.randint(-127, 128, (M, K), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    qw = torch.randint(-127, 128, (N, K), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    sx = torch.rand((M,), generator=g, device=DEV) * 1e-3
    sw = torch.rand((N,), generator=g, device=DEV) * 1e-3
    b = torch.randn((N,), generator=g, device=DEV).to(torch.bfloat16)
    acc = torch.full((M, N), 0x7f7f7f7f, dtype=torch.int32, device=DEV)
    y = torch.full((M, N), 7.0, dtype=torch.bfloat16, device=DEV)
    gemm_i8(qx, qw, sx, sw, b, acc_out=acc, out=y)
    ref = torch._int_mm(qx, qw.t())
    assert torch.equal(acc, ref)
    del acc
    yr = ((ref.float() * sx[:, None]) * sw[None, :] + b.float()[None, :]).to(torch.bfloat16)
    assert torch.equal(y, yr)


def test_gemm_no_bias_exact():
    y, acc, oy, oacc = _gemm_case(700, 384, 512, seed=3, bias=False)
    assert torch.equal(acc, oacc) and torch.equal(y, oy)


def test_gemm_gelu_within_tolerance():
    y, acc, oy, oacc = _gemm_case(4680, 8960, 1536, seed=11, gelu=True)
    assert torch.equal(acc, oacc)
    rel = (y.float() - oy.float()).norm() / oy.float().norm()
    assert rel < 1e-2, float(rel)
    assert float((y.float() - oy.float()).abs().max()) <= 2 ** -6 * float(oy.float().abs().max())


def _linear(x, qw, sw, b, flags):
    from waveforcing_amd import _lib
    M, K = x.shape
    N = qw.shape[0]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    ws_q = torch.empty((M, K), dtype=torch.int8, device=DEV)
    ws_s = torch.empty((M,), dtype=torch.float32, device=DEV)
    _lib.call("wf_w8a8_linear", x.data_ptr(), M, K, x.stride(0), qw.data_ptr(), sw.data_ptr(), b.data_ptr(), N,
              y.data_ptr(), y.stride(0), flags, ws_q.data_ptr(), ws_s.data_ptr(), _lib.stream_handle(DEV))
    return y


def test_linear_gelu_input_equals_gelu_epilogue_and_oracle():
    """fc_in -> GELU -> fc_out at the 1.3B shapes: GELU applied by fc_out's input quantizer
    (WF_LINEAR_GELU_INPUT) equals, bit for bit, GELU applied in fc_in's GEMM epilogue, and the oracle's
    F.gelu(tanh) on the bf16 fc_in output within the GELU tolerance."""
    import torch.nn.functional as F

    from waveforcing_amd import _lib
    M, D, FF = 4680, 1536, 8960
    x = inputs.outlier_activations(M, D, seed=31, chan_seed=32)
    w1, b1 = inputs.linear_weights(FF, D, w_seed=33, b_seed=34)
    w2, b2 = inputs.linear_weights(D, FF, w_seed=35, b_seed=36)
    qx, sx = _quant_rows_i8(x.to(DEV))
    q1, s1 = _quant_rows_i8(w1.to(DEV))
    q2, s2 = _quant_rows_i8(w2.to(DEV))
    pre = gemm_i8(qx, q1, sx, s1, b1.to(DEV))
    post = gemm_i8(qx, q1, sx, s1, b1.to(DEV), gelu=True)
    got = _linear(pre, q2, s2, b2.to(DEV), _lib.LINEAR_GELU_INPUT)
    want = _linear(post, q2, s2, b2.to(DEV), 0)
    assert torch.equal(got, want)
    ref = olin.i8_linear(F.gelu(pre.cpu().float(), approximate="tanh").to(torch.bfloat16), w2, b2)
    rel = (got.cpu().float() - ref.float()).norm() / ref.float().norm()
    assert rel < 1e-2, float(rel)


def test_linear_module_matches_oracle():
    x, w, b = inputs.linear_1p3b()
    lin = WaveW8A8Linear(w.to(DEV), b.to(DEV))
    y, none = lin(x.to(DEV).reshape(1, 4680, 1536))
    assert none is None and y.shape == (1, 4680, 1536)
    assert torch.equal(y.cpu().reshape(4680, 1536), olin.i8_linear(x, w, b))


def test_module_swap_scopes():
    class FFN(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.fc_in = torch.nn.Linear(64, 256)
            self.act = torch.nn.GELU(approximate="tanh")
            self.fc_out = torch.nn.Linear(256, 64)

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.q = torch.nn.Linear(64, 64)
            self.ffn = FFN()

    class T(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = torch.nn.ModuleList([Block(), Block()])

    t = T().to(DEV).to(torch.bfloat16)
    assert quantize_transformer_w8a8(t, scope="ffn") == 4
    assert isinstance(t.blocks[0].ffn.act, torch.nn.Identity) and t.blocks[0].ffn.fc_in.gelu
    t2 = T().to(DEV).to(torch.bfloat16)
    assert quantize_transformer_w8a8(t2, scope="all") == 6
    with pytest.raises(ValueError):
        quantize_transformer_w8a8(torch.nn.Linear(4, 4))


@pytest.mark.parametrize("M,N,K,pad,offset", [
    (700, 512, 256, 16, 0),     # rows strided by N + 16, 16-byte aligned: full 16-byte stores
    (700, 512, 256, 12, 4),     # an 8-byte-aligned view with an odd row stride: 8-byte stores
    (300, 1540, 128, 20, 4),    # N % 8 == 4 inside a strided view, one K step
])
def test_gemm_into_strided_views(M, N, K, pad, offset):
    """y written into a column window of a wider matrix (ldy > N, possibly 8-byte aligned only): equal to the
    oracle inside the window, the columns around it untouched."""
    x = inputs.outlier_activations(M, K, seed=N, chan_seed=N + 1)
    w, b = inputs.linear_weights(N, K, w_seed=N + 2, b_seed=N + 3)
    qx, sx = olin.i8_quant_rows(x)
    qw, sw = olin.i8_quant_rows(w)
    big = torch.full((M, N + pad), 7.0, dtype=torch.bfloat16, device=DEV)
    view = big[:, offset:offset + N]
    gemm_i8(qx.to(DEV), qw.to(DEV), sx.to(DEV), sw.to(DEV), b.to(DEV), out=view)
    oy, _ = olin.i8_gemm(qx, qw, sx, sw, b)
    got = big.cpu()
    assert torch.equal(got[:, offset:offset + N], oy)
    assert bool((got[:, :offset] == 7.0).all()) and bool((got[:, offset + N:] == 7.0).all())
