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

``WaveFp8Linear`` is the reference's own arithmetic on the e4m3 matrix
cores: one fp32 scale per weight tensor (fp8.py:33-35), one bf16-computed
scale per activation tensor at every call (fp8.py:47-48), fp32
accumulation, both scales and the bias in the epilogue (fp8.py:49-56).
``quantize_transformer_fp8`` swaps it in like the reference's function of
that name.
"""

from __future__ import annotations

import os

import torch
import torch.nn as nn

from . import _lib


def _quant_rows_i8(x2: torch.Tensor):
    """bf16 [R, K] on the GPU -> (int8 [R, K], fp32 [R]) via wf_act_quant_i8."""
    R, K = x2.shape
    q = torch.empty((R, K), dtype=torch.int8, device=x2.device)
    s = torch.empty((R,), dtype=torch.float32, device=x2.device)
    _lib.call("wf_act_quant_i8", x2.data_ptr(), R, K, x2.stride(0), q.data_ptr(), s.data_ptr(),
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


def fp8_quant_pertensor(x2: torch.Tensor, mode: int):
    """bf16 [R, K] -> (e4m3 codes [R, K] as torch.float8_e4m3fn, fp32 0-dim scale).

    ``mode`` is ``_lib.FP8_TENSOR_WEIGHT`` (fp8.py:33-35) or
    ``_lib.FP8_TENSOR_ACT`` (fp8.py:47-48)."""
    x2 = _as_bf16_rows(x2)
    R, K = x2.shape
    codes = torch.empty((R, K), dtype=torch.float8_e4m3fn, device=x2.device)
    scale = torch.empty((), dtype=torch.float32, device=x2.device)
    partials = torch.empty((_lib.FP8_AMAX_PARTIALS,), dtype=torch.float32, device=x2.device)
    _lib.call("wf_fp8_quant_pertensor", x2.data_ptr(), R, K, x2.stride(0), mode, codes.data_ptr(),
              scale.data_ptr(), partials.data_ptr(), _lib.stream_handle(x2.device))
    return codes, scale


def gemm_fp8_pertensor(a_codes, w_codes, a_scale, w_scale, bias=None, out=None):
    """y bf16 [M, N] = bf16(e4m3 a [M, K] x e4m3 w [N, K]^T * a_scale * w_scale + bias)."""
    M, K = a_codes.shape
    N = w_codes.shape[0]
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=a_codes.device)
    _lib.call("wf_gemm_fp8_pertensor", a_codes.data_ptr(), w_codes.data_ptr(), M, N, K, a_scale.data_ptr(),
              w_scale.data_ptr(), _lib.ptr(bias), y.data_ptr(), y.stride(0), _lib.stream_handle(a_codes.device))
    return y


class WaveFp8Linear(nn.Module):
    """The reference's per-tensor e4m3 W8A8 linear (wave_rt/runtime/fp8.py:21-61) on HIP.

    Same constructor and buffers (``w_fp8`` e4m3fn [out, in], ``w_scale`` fp32
    0-dim, ``bias`` in the output dtype) and the same ``(y, None)`` return.
    ``compile_fwd`` is accepted for signature parity; the forward is two
    kernel launches with nothing to trace.  Weights must be bf16 (the
    quantization kernel reads bf16; the Wan blocks are bf16).
    """

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None, compile_fwd: bool | None = None) -> None:
        super().__init__()
        if weight.dim() != 2:
            raise ValueError("weight must be 2-D [out, in]")
        if weight.dtype != torch.bfloat16:
            raise ValueError(f"WaveFp8Linear expects a bfloat16 weight, got {weight.dtype}")
        if not weight.is_cuda:
            raise ValueError("WaveFp8Linear quantizes on the GPU; move the weight to a GPU first")
        self.out_dtype = weight.dtype
        self.out_features, self.in_features = weight.shape
        if self.in_features % 16 or self.out_features % 4:
            raise ValueError(f"unsupported linear shape {tuple(weight.shape)} (in % 16, out % 4 required)")
        w_fp8, w_scale = fp8_quant_pertensor(weight.detach().contiguous(), _lib.FP8_TENSOR_WEIGHT)
        self.register_buffer("w_fp8", w_fp8)
        self.register_buffer("w_scale", w_scale)
        if bias is not None:
            self.register_buffer("bias", bias.detach().to(self.out_dtype).contiguous())
        else:
            self.bias = None
        self.compile_fwd = compile_fwd

    def _raw(self, x2: torch.Tensor) -> torch.Tensor:
        x2 = _as_bf16_rows(x2)
        M, K = x2.shape
        if K != self.in_features:
            raise ValueError(f"input width {K} != in_features {self.in_features}")
        ws_codes = torch.empty((M, K), dtype=torch.uint8, device=x2.device)
        ws_scale = torch.empty((1,), dtype=torch.float32, device=x2.device)
        ws_partials = torch.empty((_lib.FP8_AMAX_PARTIALS,), dtype=torch.float32, device=x2.device)
        y = torch.empty((M, self.out_features), dtype=torch.bfloat16, device=x2.device)
        _lib.call(
            "wf_fp8_linear_pertensor", x2.data_ptr(), M, K, x2.stride(0), self.w_fp8.data_ptr(),
            self.w_scale.data_ptr(), _lib.ptr(self.bias), self.out_features, y.data_ptr(), y.stride(0),
            ws_codes.data_ptr(), ws_scale.data_ptr(), ws_partials.data_ptr(), _lib.stream_handle(x2.device),
        )
        return y

    def forward(self, x: torch.Tensor):
        shape = x.shape
        y = self._raw(x.reshape(-1, shape[-1]))
        return y.reshape(*shape[:-1], self.out_features), None


_TARGET_SUFFIXES = ("ffn.fc_in", "ffn.fc_out")


def _is_quantizable_linear(mod: nn.Module) -> bool:
    """A 2-D ``*Linear`` not yet replaced (wave_rt/runtime/fp8.py:70-77)."""
    if isinstance(mod, (WaveW8A8Linear, WaveFp8Linear)):
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


def _resolve_scope(scope: str | None) -> str:
    return os.environ.get("WAVE_FP8_SCOPE", "ffn") if scope is None else scope


def _swap_block_linears(transformer: nn.Module, scope: str, make) -> int:
    """Replace the selected linears of every block with ``make(parent, leaf, w, b)``.

    Selection follows wave_rt/runtime/fp8.py:93-137: scope ``ffn`` (the
    default, from ``WAVE_FP8_SCOPE``) targets ``ffn.fc_in`` and ``ffn.fc_out``,
    scope ``all`` every 2-D ``*Linear`` of a block; a transformer without
    ``.blocks`` raises ValueError."""
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
            if mod is None or isinstance(mod, (WaveW8A8Linear, WaveFp8Linear)):
                continue
            w, b = _get_weight_bias(mod)
            if w is None or w.dim() != 2:
                continue
            setattr(parent, leaf, make(parent, leaf, w, b))
            n += 1
    return n


def quantize_transformer_w8a8(transformer: nn.Module, verbose: bool = False, scope: str | None = None,
                              fuse_gelu: bool = True) -> int:
    """Replace selected block linears in place with WaveW8A8Linear; return the count.

    Selection follows wave_rt/runtime/fp8.py:93-137.  With ``fuse_gelu`` a
    block whose ``ffn.act`` is ``nn.GELU(approximate='tanh')`` gets the
    activation folded into the fc_in epilogue (``ffn.act`` becomes Identity).
    """

    def make(parent, leaf, w, b):
        gelu = False
        act = getattr(parent, "act", None)
        if fuse_gelu and leaf == "fc_in" and isinstance(act, nn.GELU) and act.approximate == "tanh":
            gelu = True
            setattr(parent, "act", nn.Identity())
        return WaveW8A8Linear(w, b, gelu=gelu)

    scope = _resolve_scope(scope)
    n = _swap_block_linears(transformer, scope, make)
    if verbose:
        print(f"[wave-w8a8] quantized {n} linears to W8A8 int8 (per-token/per-channel, scope={scope})", flush=True)
    return n


def quantize_transformer_fp8(transformer: nn.Module, verbose: bool = False, scope: str | None = None) -> int:
    """Replace selected block linears in place with WaveFp8Linear; return the count.

    The reference's quantize_transformer_fp8 (wave_rt/runtime/fp8.py:93-137)
    with the same selection, return value and errors."""
    scope = _resolve_scope(scope)
    n = _swap_block_linears(transformer, scope, lambda parent, leaf, w, b: WaveFp8Linear(w, b))
    if verbose:
        print(f"[wave-fp8] quantized {n} linears to W8A8 e4m3 (per-tensor, scope={scope})", flush=True)
    return n
