"""Post-load W8A8 quantization of DiT block linears, on the HIP kernels.

Mirrors the interface of wave_rt/runtime/fp8.py: a linear replacement whose
``forward(x)`` returns the SGLang linear contract ``(y, None)``
(fp8.py:58-61), and an in-place module swap over ``transformer.blocks``
whose target set follows ``WAVE_FP8_SCOPE`` (``ffn``: ``ffn.fc_in`` and
``ffn.fc_out``; ``all``: every 2-D ``*Linear`` of a block) and which returns
the number of replaced modules (fp8.py:64-137).

``WaveW8A8Linear`` is the int8 scheme: the weight is quantized once per
output channel at construction, activations per token at every call, the
GEMM accumulates in int32 on the i8 matrix cores and the epilogue applies
both scales and the bias (optionally followed by GELU-tanh, fusing the FFN
activation into fc_in).
"""

from __future__ import annotations

import os

import torch
import torch.nn as nn

from . import _lib


def _quant_rows_i8(x2: torch.Tensor):
    """bf16 [R, K] on the GPU -> (int8 [R, K], fp32 [R]) via wf_quant_rows_i8."""
    R, K = x2.shape
    q = torch.empty((R, K), dtype=torch.int8, device=x2.device)
    s = torch.empty((R,), dtype=torch.float32, device=x2.device)
    _lib.call("wf_quant_rows_i8", x2.data_ptr(), R, K, x2.stride(0), q.data_ptr(), s.data_ptr(),
              _lib.stream_handle(x2.device))
    return q, s


def _as_bf16_rows(x: torch.Tensor) -> torch.Tensor:
    if x.dtype != torch.bfloat16:
        raise ValueError(f"expected bfloat16 activations, got {x.dtype}")
    if x.stride(-1) != 1 or (x.dim() == 2 and x.stride(0) % 8) or x.data_ptr() % 16:
        x = x.contiguous()
    return x


def gemm_i8(qx, qw, sx, sw, bias=None, gelu: bool = False, acc_out=None, out=None):
    """y bf16 [M, N] = epilogue(int8 qx [M, K] x int8 qw [N, K]^T) via wf_gemm_i8."""
    M, K = qx.shape
    N = qw.shape[0]
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=qx.device)
    _lib.call(
        "wf_gemm_i8", qx.data_ptr(), qw.data_ptr(), M, N, K, sx.data_ptr(), sw.data_ptr(),
        _lib.ptr(bias), y.data_ptr(), y.stride(0), _lib.ptr(acc_out), _lib.GEMM_GELU_TANH if gelu else 0,
        _lib.stream_handle(qx.device),
    )
    return y


class WaveW8A8Linear(nn.Module):
    """int8 W8A8 linear with the reference linear's return contract ``(y, None)``."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None, gelu: bool = False) -> None:
        super().__init__()
        if weight.dim() != 2:
            raise ValueError("weight must be 2-D [out, in]")
        if not weight.is_cuda:
            raise ValueError("WaveW8A8Linear quantizes on the GPU; move the weight to a GPU first")
        self.out_dtype = torch.bfloat16
        self.out_features, self.in_features = weight.shape
        if self.in_features % 16 or self.out_features % 4:
            raise ValueError(f"unsupported linear shape {tuple(weight.shape)} (in % 16, out % 4 required)")
        w = weight.detach().to(torch.bfloat16).contiguous()
        qw, sw = _quant_rows_i8(w)
        self.register_buffer("w_i8", qw)
        self.register_buffer("w_scale", sw)
        if bias is not None:
            self.register_buffer("bias", bias.detach().to(torch.bfloat16).contiguous())
        else:
            self.bias = None
        self.gelu = gelu

    def _raw(self, x2: torch.Tensor) -> torch.Tensor:
        x2 = _as_bf16_rows(x2)
        M, K = x2.shape
        if K != self.in_features:
            raise ValueError(f"input width {K} != in_features {self.in_features}")
        ws_q = torch.empty((M, K), dtype=torch.int8, device=x2.device)
        ws_s = torch.empty((M,), dtype=torch.float32, device=x2.device)
        y = torch.empty((M, self.out_features), dtype=torch.bfloat16, device=x2.device)
        _lib.call(
            "wf_w8a8_linear", x2.data_ptr(), M, K, x2.stride(0), self.w_i8.data_ptr(), self.w_scale.data_ptr(),
            _lib.ptr(self.bias), self.out_features, y.data_ptr(), y.stride(0),
            _lib.GEMM_GELU_TANH if self.gelu else 0, ws_q.data_ptr(), ws_s.data_ptr(),
            _lib.stream_handle(x2.device),
        )
        return y

    def forward(self, x: torch.Tensor):
        shape = x.shape
        y = self._raw(x.reshape(-1, shape[-1]))
        return y.reshape(*shape[:-1], self.out_features), None


_TARGET_SUFFIXES = ("ffn.fc_in", "ffn.fc_out")


def _is_quantizable_linear(mod: nn.Module) -> bool:
    """A 2-D ``*Linear`` not yet replaced (wave_rt/runtime/fp8.py:70-77)."""
    if isinstance(mod, WaveW8A8Linear):
        return False
    w = getattr(mod, "weight", None)
    if not isinstance(w, torch.Tensor) or w.dim() != 2:
        return False
    return type(mod).__name__.endswith("Linear")


def _get_weight_bias(mod: nn.Module):
    """[out, in] weight and optional bias (wave_rt/runtime/fp8.py:80-90)."""
    w = getattr(mod, "weight", None)
    if w is None:
        return None, None
    b = getattr(mod, "bias", None)
    if isinstance(b, nn.Parameter):
        b = b.data
    elif not isinstance(b, torch.Tensor):
        b = None
    return w.data, b


def quantize_transformer_w8a8(transformer: nn.Module, verbose: bool = False, scope: str | None = None,
                              fuse_gelu: bool = True) -> int:
    """Replace selected block linears in place with WaveW8A8Linear; return the count.

    Selection follows wave_rt/runtime/fp8.py:93-137.  With ``fuse_gelu`` a
    block whose ``ffn.act`` is ``nn.GELU(approximate='tanh')`` gets the
    activation folded into the fc_in epilogue (``ffn.act`` becomes Identity).
    """
    if scope is None:
        scope = os.environ.get("WAVE_FP8_SCOPE", "ffn")
    blocks = getattr(transformer, "blocks", None)
    if blocks is None:
        raise ValueError("transformer has no .blocks to quantize")
    n = 0
    for block in blocks:
        if scope == "all":
            targets = [name for name, m in block.named_modules() if name and _is_quantizable_linear(m)]
        else:
            targets = list(_TARGET_SUFFIXES)
        for suffix in targets:
            parent = block
            *path, leaf = suffix.split(".")
            ok = True
            for p in path:
                parent = getattr(parent, p, None)
                if parent is None:
                    ok = False
                    break
            if not ok:
                continue
            mod = getattr(parent, leaf, None)
            if mod is None or isinstance(mod, WaveW8A8Linear):
                continue
            w, b = _get_weight_bias(mod)
            if w is None or w.dim() != 2:
                continue
            gelu = False
            act = getattr(parent, "act", None)
            if fuse_gelu and leaf == "fc_in" and isinstance(act, nn.GELU) and act.approximate == "tanh":
                gelu = True
                setattr(parent, "act", nn.Identity())
            setattr(parent, leaf, WaveW8A8Linear(w, b, gelu=gelu))
            n += 1
    if verbose:
        print(f"[wave-w8a8] quantized {n} linears to W8A8 int8 (per-token/per-channel, scope={scope})", flush=True)
    return n
