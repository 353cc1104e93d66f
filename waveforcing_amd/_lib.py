"""ctypes binding of libwf_mi355x.so (the C ABI declared in include/wf_api.h).

Every call goes through :func:`call`, which turns a non-zero status into a
``RuntimeError`` carrying the library's thread-local message, the same way the
reference's driver wrapper turns CUDA driver errors into ``RuntimeError``
(wave_rt/distributed/ipc.py:28-37).  There is no fallback: if the library is
missing or fails to load, every operation raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libwf_mi355x.so")

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float

# name -> argtypes; pointers are passed as integers (device addresses).
SIGNATURES: dict[str, list] = {
    "wf_abi_version": [],
    "wf_last_error": [],
    "wf_fp8_e4m3_encode_f32": [_c_void_p, _c_void_p, _i64, _c_void_p],
    "wf_fp8_e4m3_decode_f32": [_c_void_p, _c_void_p, _i64, _c_void_p],
    "wf_fp8_kv_pack": [
        _c_void_p, _c_void_p, _i64, _i32, _i32, _i64,
        _c_void_p, _i64, _i32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
        _c_void_p,
    ],
    "wf_fp8_kv_pack_rope": [
        _c_void_p, _c_void_p, _i64, _i32, _i32, _i64,
        _c_void_p, _c_void_p,
        _c_void_p, _i64, _i32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
        _c_void_p,
    ],
    "wf_fp8_kv_pack_rope_tiled": [
        _c_void_p, _c_void_p, _i64, _i32, _i32, _i64,
        _c_void_p, _c_void_p, _i64,
        _c_void_p, _i64, _i32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
        _c_void_p,
    ],
    "wf_k_norm_rope_kv_pack": [
        _c_void_p, _c_void_p, _i64, _i32, _i32, _i64,
        _f32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
        _c_void_p, _i64, _i32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
        _c_void_p,
    ],
    "wf_qk_norm_rope_kv_pack": [
        _c_void_p, _i64, _c_void_p,
        _c_void_p, _c_void_p, _i64, _i32, _i32, _i64,
        _f32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
        _c_void_p, _i64, _i32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
        _c_void_p,
    ],
    "wf_fp8_kv_unpack": [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
        _c_void_p, _i64, _i32, _i64, _i32, _i32,
        _c_void_p, _c_void_p,
        _c_void_p,
    ],
    "wf_act_quant_i8": [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p],
    "wf_flow_add_noise_bf16": [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i32, _f32, _c_void_p, _c_void_p],
    "wf_gemm_i8": [
        _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
        _c_void_p, _i64, _c_void_p, _i32, _c_void_p,
    ],
    "wf_w8a8_linear": [
        _c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
        _i64, _c_void_p, _i64, _i32, _c_void_p, _c_void_p, _c_void_p,
    ],
    "wf_w8a8_linear_static": [
        _c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
        _i64, _c_void_p, _i64, _i32, _c_void_p,
    ],
    "wf_fp8_quant_pertensor": [_c_void_p, _i64, _i64, _i64, _i32, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "wf_fp8_dequant_pertensor_f32": [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p],
    "wf_gemm_fp8_pertensor": [
        _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p,
    ],
    "wf_fp8_linear_pertensor": [
        _c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p,
    ],
    "wf_attn_paged_fp8": [
        _c_void_p, _i64, _i32, _i32, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _i64, _i32, _c_void_p, _i64, _i64, _f32, _c_void_p, _i64, _c_void_p,
    ],
    "wf_attn_paged_fp8_qk8": [
        _c_void_p, _i64, _i32, _i32, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _i64, _i32, _c_void_p, _i64, _i64, _f32, _c_void_p, _i64, _c_void_p,
    ],
    "wf_attn_paged_fp8_qkpv8": [
        _c_void_p, _i64, _i32, _i32, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _i64, _i32, _c_void_p, _i64, _i64, _f32, _c_void_p, _i64, _c_void_p,
    ],
    "wf_attn_dense_bf16": [
        _c_void_p, _i64, _i32, _i32, _i64, _c_void_p, _c_void_p, _i64, _i64, _f32, _c_void_p, _i64, _c_void_p,
    ],
    "wf_ln_modulate_quant": [
        _c_void_p, _i64, _i32, _i64, _f32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32,
        _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,
    ],
    "wf_gate_residual_ln_quant": [
        _c_void_p, _i64, _i32, _i64, _c_void_p, _i64, _c_void_p, _i64, _f32, _c_void_p, _c_void_p,
        _c_void_p, _c_void_p, _i64, _i32, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,
    ],
    "wf_rmsnorm_rope": [
        _c_void_p, _i64, _i32, _i64, _i32, _f32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p,
    ],
    "wf_gemm_bf16": [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i32, _c_void_p],
    "wf_patchify_bf16": [_c_void_p, _i64, _i32, _i32, _i32, _i32, _c_void_p, _c_void_p],
    "wf_unpatchify_flow_x0_bf16": [_c_void_p, _c_void_p, _i64, _i32, _i32, _i32, _i32, ctypes.c_double, _c_void_p,
                                   _c_void_p],
    "wf_gate_residual": [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64, _i32, _i32, _c_void_p],
}

GEMM_GELU_TANH = 1
LINEAR_GELU_INPUT = 2
FP8_TENSOR_WEIGHT = 0
FP8_TENSOR_ACT = 1
FP8_AMAX_PARTIALS = 1024
BF16_SILU_IN = 1
BF16_SILU_OUT = 2
BF16_GELU_OUT = 4
W8A8_STATIC_MAX_CODES = 64 << 20
W8A8_STATIC_MAX_ROWS = 65536

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class NativeLibraryMissing(RuntimeError):
    """The HIP library has not been built (run ``python -m waveforcing_amd.build``)."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library with argument types installed."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryMissing(
                f"{LIB_PATH} not found; build it with `python -m waveforcing_amd.build`"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_char_p if name == "wf_last_error" else ctypes.c_int
        _lib = lib
        return lib


def last_error() -> str:
    return load().wf_last_error().decode(errors="replace")


_fns: dict = {}


def call(name: str, *args) -> None:
    """Invoke ``name`` and raise ``RuntimeError`` on a non-zero status."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(load(), name)
    status = fn(*args)
    if status != 0:
        raise RuntimeError(f"{name} failed (status {status}): {last_error()}")


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_handle(device=None) -> int:
    """hipStream_t of torch's current stream on ``device`` (None, an index, a name or a torch.device)."""
    import torch

    if isinstance(device, torch.device) and device.type == "cuda" and device.index is not None:
        return torch._C._cuda_getCurrentRawStream(device.index)
    return torch.cuda.current_stream(device).cuda_stream
