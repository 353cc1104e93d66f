"""GPU parity of the reference's per-tensor e4m3 W8A8 linear (WaveFp8Linear,
wave_rt/runtime/fp8.py:21-61) against the CPU oracle.

Bars: e4m3 codes and fp32 scales bit-exact (weights in fp32 arithmetic,
activations in bf16 tensor arithmetic); GEMM output within 1e-2 relative
error (the stated tolerance; the fp32 accumulation order of the matrix
cores differs from torch's CPU _scaled_mm).
"""

import pytest
import torch

from oracle import linear as olin
from waveforcing_amd import _lib, inputs
from waveforcing_amd.fp8 import (WaveFp8Linear, fp8_quant_pertensor, gemm_fp8_pertensor,
                                 quantize_transformer_fp8)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _codes(t):
    return t.cpu().view(torch.uint8)


@pytest.mark.parametrize("R,K,seed", [(1536, 1536, 0), (8960, 1536, 1), (1, 8, 2), (37, 48, 3), (300, 8960, 4)])
def test_weight_quant_bit_exact(R, K, seed):
    w, _ = inputs.linear_weights(R, K, w_seed=seed, b_seed=seed + 1)
    codes, scale = fp8_quant_pertensor(w.to(DEV), _lib.FP8_TENSOR_WEIGHT)
    ocodes, oscale = olin.fp8_quant_weight(w)
    assert torch.equal(scale.cpu(), oscale)
    assert torch.equal(_codes(codes), ocodes.view(torch.uint8))


@pytest.mark.parametrize("M,K,seed", [(4680, 1536, 0), (4680, 8960, 1), (1, 8, 2), (513, 272, 3)])
def test_activation_quant_bit_exact(M, K, seed):
    x = inputs.outlier_activations(M, K, seed=seed, chan_seed=seed + 7)
    codes, scale = fp8_quant_pertensor(x.to(DEV), _lib.FP8_TENSOR_ACT)
    ocodes, oscale = olin.fp8_quant_act(x)
    assert torch.equal(scale.cpu(), oscale.float())
    assert torch.equal(_codes(codes), ocodes.view(torch.uint8))


def test_activation_quant_special_values():
    """All-zero input takes the bf16(1e-8) scale floor; tiny inputs hit the
    floor with subnormal codes; a row of the largest bf16 values saturates
    at 448 only through the bf16-rounded scale."""
    zero = torch.zeros((16, 64), dtype=torch.bfloat16)
    tiny = torch.full((4, 32), 3e-10, dtype=torch.bfloat16)
    tiny[0, 0] = 2e-9
    big = (torch.linspace(-1.0, 1.0, 8 * 64) * 3.3e38).reshape(8, 64).to(torch.bfloat16)
    assert torch.isfinite(big.float()).all()
    for x in (zero, tiny, big):
        codes, scale = fp8_quant_pertensor(x.to(DEV), _lib.FP8_TENSOR_ACT)
        ocodes, oscale = olin.fp8_quant_act(x)
        assert torch.equal(scale.cpu(), oscale.float())
        assert torch.equal(_codes(codes), ocodes.view(torch.uint8))


def test_strided_rows_quantize_like_contiguous():
    x = inputs.outlier_activations(256, 512, seed=5, chan_seed=6)
    wide = torch.zeros((256, 640), dtype=torch.bfloat16)
    wide[:, :512] = x
    c1, s1 = fp8_quant_pertensor(wide.to(DEV)[:, :512], _lib.FP8_TENSOR_ACT)
    c2, s2 = fp8_quant_pertensor(x.to(DEV), _lib.FP8_TENSOR_ACT)
    assert torch.equal(s1, s2) and torch.equal(_codes(c1), _codes(c2))


def _rel(y, ref):
    return float((y.float() - ref.float()).norm() / ref.float().norm())


@pytest.mark.parametrize("M,N,K", [
    (4680, 1536, 1536), (4680, 8960, 1536), (4680, 1536, 8960),
    (1, 4, 16), (17, 132, 48), (300, 256, 1552), (513, 1540, 272),
])
def test_gemm_within_tolerance(M, N, K):
    seed = M + N + K
    x = inputs.outlier_activations(M, K, seed=seed, chan_seed=seed + 1)
    w, b = inputs.linear_weights(N, K, w_seed=seed + 2, b_seed=seed + 3)
    xc, xs = olin.fp8_quant_act(x)
    wc, ws = olin.fp8_quant_weight(w)
    y = gemm_fp8_pertensor(xc.to(DEV), wc.to(DEV), xs.float().reshape(1).to(DEV), ws.reshape(1).to(DEV), b.to(DEV))
    ref = torch._scaled_mm(xc, wc.t(), scale_a=xs.reshape(()).float(), scale_b=ws, bias=b, out_dtype=torch.bfloat16)
    # products of e4m3 codes are exact in fp32: check against a float64 sum too
    exact = (xc.double() @ wc.double().t()) * float(xs) * float(ws) + b.double()
    assert _rel(y.cpu(), ref) < 1e-2
    assert _rel(y.cpu(), exact) < 1e-2
    assert float((y.cpu().double() - exact).abs().max()) <= 2 ** -7 * float(exact.abs().max()) + 1e-6


def test_linear_module_matches_reference_linear():
    x, w, b = inputs.linear_1p3b()
    lin = WaveFp8Linear(w.to(DEV), b.to(DEV))
    assert lin.w_fp8.dtype == torch.float8_e4m3fn and lin.w_scale.dim() == 0 and lin.bias.dtype == torch.bfloat16
    y, none = lin(x.to(DEV).reshape(1, 4680, 1536))
    assert none is None and y.shape == (1, 4680, 1536)
    wf, wscale = olin.fp8_quant_weight(w)
    assert torch.equal(lin.w_scale.cpu(), wscale) and torch.equal(_codes(lin.w_fp8), wf.view(torch.uint8))
    ref = olin.fp8_linear(x, wf, wscale, b)
    assert _rel(y.cpu().reshape(4680, 1536), ref) < 1e-2


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
    assert quantize_transformer_fp8(t, scope="ffn") == 4
    assert isinstance(t.blocks[0].ffn.fc_in, WaveFp8Linear)
    assert isinstance(t.blocks[0].ffn.act, torch.nn.GELU)  # the reference keeps the activation module
    assert quantize_transformer_fp8(t, scope="ffn") == 0   # already replaced
    t2 = T().to(DEV).to(torch.bfloat16)
    assert quantize_transformer_fp8(t2, scope="all") == 6
    with pytest.raises(ValueError):
        quantize_transformer_fp8(torch.nn.Linear(4, 4))
