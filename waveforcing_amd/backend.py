"""Attention-backend registry and the patched self-attention step.

Mirrors the process-global state and backend switches of
wave_rt/runtime/backend.py:18-62 (``_WAVE_STATE``, ``set_exchange_fn``,
``enable_fa_custom``/``enable_sage``) and the attention part of its patched
``CausalWanSelfAttention.forward`` (backend.py:102-157): RoPE'd q/k go to the
installed exchange closure, which returns the context, then the selected
attention kernel runs non-causally over it.

The HIP backend, ``hip_fp8``, takes the context as a page descriptor
(:class:`waveforcing_amd.kv.PagedKV`) that the paged FP8 exchange returns in
place of the dense ``Kb[:active_len]`` views (paged.py:246-247), and runs
``wf_attn_paged_fp8`` on it.  ``hip_fp8_qk`` is the quantized-QK counterpart
of the reference's SageAttention backend (``enable_sage``, backend.py:57-62,
144-146): the same call over the same pages through ``wf_attn_paged_fp8_qk8``,
which quantizes each query to e4m3 and runs QK^T on the fp8 matrix cores
against the pages' K codes, with V exact; approximate by design, like Sage.
``hip_fp8_qkpv`` (``wf_attn_paged_fp8_qkpv8``) also runs P.V on the fp8 matrix
cores, against the pages' V codes, as Sage's fp8 P.V product does.
"""

from __future__ import annotations

import math
import time
from typing import Callable

import torch

from . import _lib
from .kv import PagedKV

ATTENTION_BACKENDS = ("torch_sdpa", "fa_custom", "sa", "fa", "fa2", "hip_fp8", "hip_fp8_qk", "hip_fp8_qkpv")

_WAVE_STATE: dict = {
    "exchange_fn": None,
    "attn": "torch_sdpa",
    "fa_func": None,
    "layer_prof_sink": None,
}


def set_exchange_fn(fn: Callable | None) -> None:
    _WAVE_STATE["exchange_fn"] = fn


def set_layer_prof_sink(sink) -> None:
    """Set the optional sink for attention completion events."""
    _WAVE_STATE["layer_prof_sink"] = sink


def prof_reset(on: bool) -> None:
    _WAVE_STATE["prof"] = on
    _WAVE_STATE["attn_ms"] = 0.0
    _WAVE_STATE["exch_ms"] = 0.0


def prof_read() -> tuple:
    return (_WAVE_STATE.get("attn_ms", 0.0), _WAVE_STATE.get("exch_ms", 0.0), _WAVE_STATE.get("klen", 0))


def attn_paged_fp8(q: torch.Tensor, k: PagedKV, v: PagedKV | None = None, causal: bool = False,
                   softmax_scale: float | None = None, out: torch.Tensor | None = None,
                   quantized_qk: bool = False, fp8_pv: bool = False) -> torch.Tensor:
    """flash_attn_func-shaped call: q [1, Lq, H, D] (or [Lq, H, D]) bf16 over a paged FP8 context.

    ``k`` carries both pools; ``v`` is accepted for call compatibility and
    must be ``k`` itself or None.  Returns bf16 with q's shape.  With
    ``quantized_qk`` the scores come from e4m3 queries against the K codes
    on the fp8 matrix cores (wf_attn_paged_fp8_qk8); ``fp8_pv`` (which implies
    it) runs P.V there too, against the V codes (wf_attn_paged_fp8_qkpv8).
    """
    if causal:
        raise ValueError("the wavefront attention is non-causal over the context (backend.py:141-148)")
    if not isinstance(k, PagedKV) or (v is not None and v is not k):
        raise TypeError("hip_fp8 attention takes the PagedKV descriptor returned by the paged exchange")
    squeeze = q.dim() == 4
    q3 = q[0] if squeeze else q
    if q3.dim() != 3 or q3.dtype != torch.bfloat16:
        raise ValueError(f"q must be bf16 [1, Lq, H, D] or [Lq, H, D], got {tuple(q.shape)} {q.dtype}")
    Lq, H, D = q3.shape
    pool = k.pool
    if H != pool.n_heads or D != pool.head_dim:
        raise ValueError(f"q heads/dim ({H}, {D}) differ from the pool ({pool.n_heads}, {pool.head_dim})")
    if q3.stride(2) != 1 or q3.stride(1) != D or q3.data_ptr() % 16 or q3.stride(0) % 8:
        q3 = q3.contiguous()
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    o = out if out is not None else torch.empty((Lq, H, D), dtype=torch.bfloat16, device=q3.device)
    if o.dim() == 4:
        o = o[0]
    entry = "wf_attn_paged_fp8_qkpv8" if fp8_pv else "wf_attn_paged_fp8_qk8" if quantized_qk else "wf_attn_paged_fp8"
    _lib.call(
        entry, q3.data_ptr(), Lq, H, D, q3.stride(0),
        pool.k_codes.data_ptr(), pool.v_codes.data_ptr(), pool.k_scales.data_ptr(), pool.v_scales.data_ptr(),
        pool.pool_pages, pool.page_tokens, k.table.dev.data_ptr(), len(k.table), k.n_tokens,
        float(softmax_scale), o.data_ptr(), o.stride(0), _lib.stream_handle(q3.device),
    )
    return o.unsqueeze(0) if squeeze else o


def attn_dense_bf16(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, softmax_scale: float | None = None,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """Non-causal attention of q [Lq, H, D] over dense bf16 k, v [Lk, H, D] (text cross-attention)."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dim() != 3 or t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bf16 [L, H, D], got {tuple(t.shape)} {t.dtype}")
    Lq, H, D = q.shape
    if k.shape != v.shape or k.shape[1:] != (H, D):
        raise ValueError("k/v shapes must match and agree with q's heads and head_dim")

    def rows(t):
        if t.stride(2) != 1 or t.stride(1) != D or t.stride(0) % 8 or t.data_ptr() % 16:
            t = t.contiguous()
        return t

    q, k, v = rows(q), rows(k), rows(v)
    if k.stride(0) != v.stride(0):
        k, v = k.contiguous(), v.contiguous()
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    o = out if out is not None else torch.empty((Lq, H, D), dtype=torch.bfloat16, device=q.device)
    _lib.call("wf_attn_dense_bf16", q.data_ptr(), Lq, H, D, q.stride(0), k.data_ptr(), v.data_ptr(), k.shape[0],
              k.stride(0), float(softmax_scale), o.data_ptr(), o.stride(0), _lib.stream_handle(q.device))
    return o


def attn_paged_fp8_qk(q: torch.Tensor, k: PagedKV, v: PagedKV | None = None, causal: bool = False,
                      softmax_scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """The quantized-QK form of :func:`attn_paged_fp8` (the ``fa_func`` of ``hip_fp8_qk``)."""
    return attn_paged_fp8(q, k, v, causal, softmax_scale, out, quantized_qk=True)


def attn_paged_fp8_qkpv(q: torch.Tensor, k: PagedKV, v: PagedKV | None = None, causal: bool = False,
                        softmax_scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """The quantized-QK form with the fp8 P.V product (the ``fa_func`` of ``hip_fp8_qkpv``)."""
    return attn_paged_fp8(q, k, v, causal, softmax_scale, out, fp8_pv=True)


def enable_hip_fp8() -> None:
    """Use the gfx950 paged-FP8 attention on the wavefront path."""
    _WAVE_STATE["attn"] = "hip_fp8"
    _WAVE_STATE["fa_func"] = attn_paged_fp8


def enable_hip_fp8_qk() -> None:
    """Use the quantized-QK paged-FP8 attention on the wavefront path, as ``enable_sage`` selects
    SageAttention (backend.py:57-62): e4m3 queries against the pages' K codes on the fp8 matrix cores."""
    _WAVE_STATE["attn"] = "hip_fp8_qk"
    _WAVE_STATE["fa_func"] = attn_paged_fp8_qk


def enable_hip_fp8_qkpv() -> None:
    """Use the paged-FP8 attention with both products on the fp8 matrix cores (e4m3 queries against the K
    codes; e4m3 weights p s_v against the V codes), the form of SageAttention's fp8 P.V kernels."""
    _WAVE_STATE["attn"] = "hip_fp8_qkpv"
    _WAVE_STATE["fa_func"] = attn_paged_fp8_qkpv


def paged_attention():
    """The paged attention the blocks run: the quantized form that ``hip_fp8_qk`` or ``hip_fp8_qkpv`` selects,
    the exact form otherwise."""
    return {"hip_fp8_qk": attn_paged_fp8_qk, "hip_fp8_qkpv": attn_paged_fp8_qkpv}.get(_WAVE_STATE["attn"],
                                                                                    attn_paged_fp8)


def attend(roped_query, ctx_k, ctx_v, sdpa: Callable | None = None):
    """Attention dispatch of the patched forward (backend.py:141-148)."""
    attn = _WAVE_STATE["attn"]
    if attn in ("hip_fp8", "hip_fp8_qk", "hip_fp8_qkpv"):
        return _WAVE_STATE["fa_func"](roped_query, ctx_k, ctx_v, causal=False)
    if attn == "fa_custom":
        return _WAVE_STATE["fa_func"](roped_query, ctx_k, ctx_v, causal=False)
    if attn == "sa":
        return _WAVE_STATE["fa_func"](roped_query, ctx_k, ctx_v, tensor_layout="NHD", is_causal=False)
    if sdpa is None:
        raise RuntimeError(f"attention backend {attn!r} needs the model's own attention callable")
    return sdpa(roped_query, ctx_k, ctx_v)


def exchange_and_attend(layer_idx: int, roped_query, roped_key, unroped_key, value, sdpa: Callable | None = None,
                        **geometry):
    """The body of the patched self-attention after RoPE (backend.py:122-157)."""
    exch = _WAVE_STATE["exchange_fn"]
    if exch is None:
        raise RuntimeError("no exchange function installed (set_exchange_fn)")
    profiled = bool(_WAVE_STATE.get("prof"))
    if profiled:
        torch.cuda.synchronize()
        started = time.perf_counter()
    ctx_k, ctx_v = exch(layer_idx=layer_idx, roped_query=roped_query, roped_key=roped_key,
                        unroped_key=unroped_key, value=value, **geometry)
    if profiled:
        torch.cuda.synchronize()
        _WAVE_STATE["exch_ms"] = _WAVE_STATE.get("exch_ms", 0.0) + (time.perf_counter() - started) * 1000
        started = time.perf_counter()
    out = attend(roped_query, ctx_k, ctx_v, sdpa)
    if profiled:
        torch.cuda.synchronize()
        _WAVE_STATE["attn_ms"] = _WAVE_STATE.get("attn_ms", 0.0) + (time.perf_counter() - started) * 1000
        _WAVE_STATE["klen"] = ctx_k.shape[1]
    sink = _WAVE_STATE.get("layer_prof_sink")
    if sink is not None:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        sink.append(ev)
    return out

