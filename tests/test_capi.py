"""C ABI checks that need no GPU: the library loads, exports every entry
point declared in include/wf_api.h, and rejects bad arguments with a status
and message before touching the device."""

import ctypes
import os
import re

import pytest

from waveforcing_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "wf_api.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(wf_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert "wf_fp8_kv_pack" in names and len(names) >= 6
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_abi_version():
    assert _lib.load().wf_abi_version() >> 16 == 1


def test_bad_head_dim_is_rejected():
    with pytest.raises(RuntimeError, match="head_dim=64"):
        _lib.call("wf_fp8_kv_pack", 1, 2, 10, 2, 64, 128, 3, 1, 16, 4, 5, 6, 7, 4, None)


def test_short_page_table_is_rejected():
    with pytest.raises(RuntimeError, match="page table covers"):
        _lib.call("wf_fp8_kv_pack", 16, 32, 100, 2, 128, 256, 48, 1, 16, 64, 80, 96, 112, 4, None)


def test_negative_size_is_rejected():
    with pytest.raises(RuntimeError, match="negative"):
        _lib.call("wf_fp8_kv_unpack", 16, 32, 48, 64, 4, 80, 1, 16, -1, 2, 128, 96, 112, None)


def test_unaligned_pointer_is_rejected():
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        _lib.call("wf_fp8_kv_pack", 17, 32, 10, 2, 128, 256, 48, 1, 16, 64, 80, 96, 112, 4, None)


def test_last_error_is_thread_local_text():
    with pytest.raises(RuntimeError):
        _lib.call("wf_fp8_e4m3_encode_f32", 0, 0, -5, None)
    assert "n=-5" in _lib.last_error()


def test_fp8_pertensor_argument_errors():
    with pytest.raises(RuntimeError, match="unknown mode"):
        _lib.call("wf_fp8_quant_pertensor", 16, 4, 64, 64, 7, 32, 48, 64, None)
    with pytest.raises(RuntimeError, match="empty tensor"):
        _lib.call("wf_fp8_quant_pertensor", 16, 0, 64, 64, 0, 32, 48, 64, None)
    with pytest.raises(RuntimeError, match="multiple of 16"):
        _lib.call("wf_gemm_fp8_pertensor", 16, 32, 4, 4, 24, 48, 64, None, 80, 4, None)
    with pytest.raises(RuntimeError, match="null pointer"):
        _lib.call("wf_fp8_linear_pertensor", 16, 4, 32, 32, 48, 64, None, 8, 80, 8, 96, None, 112, None)


def test_row_kernels_refuse_launches_beyond_2_to_32_threads():
    with pytest.raises(RuntimeError, match="too large"):
        _lib.call("wf_gate_residual", 16, 1536, 32, 1536, None, 0, 1 << 40, 1536, 4680, None)
    with pytest.raises(RuntimeError, match="too large"):
        _lib.call("wf_rmsnorm_rope", 16, 1 << 24, 1536, 1536, 128, 1e-6, 48, None, None, 64, 1536, None)
    with pytest.raises(RuntimeError, match="too large"):
        _lib.call("wf_ln_modulate_quant", 16, 1 << 24, 1536, 1536, 1e-6, None, None, None, None, 0, 4680, 32, 1536,
                  None, None, None)


def test_index_kernels_refuse_launches_beyond_2_to_32_threads():
    # one thread per item: 2^32 items or more, and sizes whose product overflows int64, are refused
    with pytest.raises(RuntimeError, match="below 2\\^32"):
        _lib.call("wf_patchify_bf16", 16, 1 << 20, 16, 3, 60, 104, 32, None)
    with pytest.raises(RuntimeError, match="below 2\\^32"):
        _lib.call("wf_patchify_bf16", 16, 1 << 40, 1 << 30, 1 << 30, 1 << 30, 1 << 30, 32, None)
    with pytest.raises(RuntimeError, match="below 2\\^32"):
        _lib.call("wf_unpatchify_flow_x0_bf16", 16, 32, 1 << 20, 16, 3, 60, 104, 0.5, 48, None)


def test_gemm_sizes_that_overflow_int64_are_refused():
    with pytest.raises(RuntimeError, match="2 GiB"):
        _lib.call("wf_gemm_i8", 16, 32, 1 << 62, 16, 1 << 62, 48, 64, None, 80, 16, None, 0, None)
    with pytest.raises(RuntimeError, match="2 GiB"):
        _lib.call("wf_w8a8_linear", 16, 1 << 40, 1 << 40, 1 << 40, 32, 48, None, 16, 80, 16, 0, 96, 112, None)


def test_pertensor_dequant_and_qk8_argument_errors():
    with pytest.raises(RuntimeError, match="multiple of 16"):
        _lib.call("wf_fp8_dequant_pertensor_f32", 16, 32, 40, 48, None)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        _lib.call("wf_fp8_dequant_pertensor_f32", 17, 32, 64, 48, None)
    with pytest.raises(RuntimeError, match="head_dim=64"):
        _lib.call("wf_attn_paged_fp8_qk8", 16, 4, 2, 64, 128, 32, 48, 64, 80, 4, 64, 96, 1, 64, 0.1, 112, 128, None)
    with pytest.raises(RuntimeError, match="wf_attn_paged_fp8_qkpv8: head_dim=64"):
        _lib.call("wf_attn_paged_fp8_qkpv8", 16, 4, 2, 64, 128, 32, 48, 64, 80, 4, 64, 96, 1, 64, 0.1, 112, 128,
                  None)
    with pytest.raises(RuntimeError, match="page_tokens=32 must be >= 64"):
        _lib.call("wf_attn_paged_fp8_qkpv8", 16, 4, 2, 128, 256, 32, 48, 64, 80, 4, 32, 96, 4, 64, 0.1, 112, 256,
                  None)
