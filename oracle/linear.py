"""W8A8 linear oracle (torch CPU).

Two schemes:

* ``fp8_*`` -- the reference's WaveFp8Linear, restated line for line from
  wave_rt/runtime/fp8.py:24-56: static per-tensor e4m3 weight quantization in
  fp32 (:33-35), dynamic per-tensor activation quantization in bf16
  arithmetic (:47-48), ``torch._scaled_mm`` with fp32 accumulation, both
  scales and the bias, bf16 out (:49-56).
* ``i8_*`` -- the workload's per-token / per-output-channel symmetric int8
  counterpart: the same clamp(min=1e-8) floor, a 127 range, round half to
  even, exact int32 accumulation (``torch._int_mm``), and the epilogue
  ``bf16((float(acc) * sx[m]) * sw[n] + bias[n])`` evaluated in that order in
  fp32.  The FFN's GELU(approximate='tanh') (naive_rt/rolling_forcing/wan/
  modules/causal_model.py:342-344) acts on the bf16 linear output.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

FP8 = torch.float8_e4m3fn
E4M3_MAX = 448.0
I8_MAX = 127.0


# ---------------------------------------------------------------- int8 scheme
def i8_quant_rows(x: torch.Tensor):
    """x [R, K] (bf16/fp32) -> (q int8 [R, K], s fp32 [R])."""
    xf = x.float()
    s = (xf.abs().amax(dim=-1) / I8_MAX).clamp(min=1e-8)
    q = torch.round(xf / s[:, None]).clamp(-I8_MAX, I8_MAX).to(torch.int8)
    return q, s


def i8_gemm(qx, qw, sx, sw, bias=None, gelu: bool = False):
    """-> (y bf16 [M, N], acc int32 [M, N])."""
    acc = torch._int_mm(qx, qw.t())
    y = acc.float() * sx[:, None]
    y = y * sw[None, :]
    if bias is not None:
        y = y + bias.float()[None, :]
    y = y.to(torch.bfloat16)
    if gelu:
        y = F.gelu(y.float(), approximate="tanh").to(torch.bfloat16)
    return y, acc


def i8_linear(x, w, bias=None, gelu: bool = False):
    """Full int8 W8A8 linear of bf16 x [M, K] with bf16 weight [N, K]."""
    qx, sx = i8_quant_rows(x)
    qw, sw = i8_quant_rows(w)
    y, _ = i8_gemm(qx, qw, sx, sw, bias, gelu)
    return y


# ---------------------------------------------------------- reference FP8
def fp8_quant_weight(weight: torch.Tensor):
    """wave_rt/runtime/fp8.py:33-35 -> (w_fp8 [N, K], w_scale fp32 0-dim)."""
    w = weight.detach().to(torch.float32)
    w_scale = (w.abs().amax() / E4M3_MAX).clamp(min=1e-8)
    return (w / w_scale).to(FP8), w_scale.reshape(()).to(torch.float32)


def fp8_quant_act(x2: torch.Tensor):
    """wave_rt/runtime/fp8.py:47-48 (bf16 arithmetic) -> (x_fp8, a_scale bf16 0-dim)."""
    a_scale = (x2.abs().amax() / E4M3_MAX).clamp(min=1e-8)
    return (x2 / a_scale).to(FP8), a_scale


def fp8_linear(x2, w_fp8, w_scale, bias=None, out_dtype=torch.bfloat16):
    """wave_rt/runtime/fp8.py:46-56."""
    x_fp8, a_scale = fp8_quant_act(x2)
    return torch._scaled_mm(
        x_fp8,
        w_fp8.t(),
        scale_a=a_scale.reshape(()).to(torch.float32),
        scale_b=w_scale,
        bias=bias,
        out_dtype=out_dtype,
    )
