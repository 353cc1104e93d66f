"""wf_w8a8_linear_static (the W8A8 linear on the library's static per-GPU
workspace) against wf_w8a8_linear (caller-passed workspace), both called
through the C ABI: equal bf16 outputs, bit for bit, on consecutive calls --
the 14B fc_out shape (m * k = 64.7 M codes, near the workspace limit), then
smaller calls that reuse the same workspace, one of them with the FFN's
GELU(tanh) applied in the input quantizer (the 1.3B fc_out) -- and the size
limits refused before any device work, including products of sizes that
overflow int64."""

import pytest
import torch

from waveforcing_amd import _lib, inputs
from waveforcing_amd.fp8 import _quant_rows_i8

DEV = "cuda:0"


def _run(name, x, qw, sw, b, flags):
    M, K = x.shape
    N = qw.shape[0]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    args = [x.data_ptr(), M, K, x.stride(0), qw.data_ptr(), sw.data_ptr(), b.data_ptr(), N, y.data_ptr(),
            y.stride(0), flags]
    if name == "wf_w8a8_linear":
        q = torch.empty((M, K), dtype=torch.int8, device=DEV)
        s = torch.empty((M,), dtype=torch.float32, device=DEV)
        args += [q.data_ptr(), s.data_ptr()]
    _lib.call(name, *args, _lib.stream_handle(DEV))
    return y


@pytest.mark.gpu
def test_static_workspace_linear_equals_workspace_linear_on_consecutive_calls():
    cases = [(4680, 5120, 13824, 0),                          # 14B fc_out: 64.7 M activation codes
             (4680, 8960, 1536, _lib.GEMM_GELU_TANH),         # 1.3B fc_in with GELU in the epilogue, smaller
             (4680, 1536, 8960, _lib.LINEAR_GELU_INPUT),      # 1.3B fc_out, GELU in the input quantizer
             (300, 1536, 512, 0)]                             # smaller still
    for i, (M, N, K, flags) in enumerate(cases):
        x = inputs.outlier_activations(M, K, seed=80 + i, chan_seed=90 + i).to(DEV)
        w, b = inputs.linear_weights(N, K, w_seed=100 + i, b_seed=110 + i)
        qw, sw = _quant_rows_i8(w.to(DEV))
        want = _run("wf_w8a8_linear", x, qw, sw, b.to(DEV), flags)
        got = _run("wf_w8a8_linear_static", x, qw, sw, b.to(DEV), flags)
        torch.cuda.synchronize()
        print(f"call {i}: m={M} n={N} k={K} flags={flags}", flush=True)
        assert torch.equal(got, want), f"call {i}"


def test_static_workspace_limits_are_refused_before_device_work():
    # m * k one row of codes past the limit, and more rows than scales; no pointer is touched
    k = 16400
    m = _lib.W8A8_STATIC_MAX_CODES // k + 1
    with pytest.raises(RuntimeError, match="static workspace"):
        _lib.call("wf_w8a8_linear_static", 16, m, k, k, 32, 48, None, 64, 80, 64, 0, None)
    with pytest.raises(RuntimeError, match="static workspace"):
        _lib.call("wf_w8a8_linear_static", 16, _lib.W8A8_STATIC_MAX_ROWS + 1, 16, 16, 32, 48, None, 64, 80, 64, 0,
                  None)
    # sizes whose products overflow int64 are refused, not wrapped
    with pytest.raises(RuntimeError, match="static workspace"):
        _lib.call("wf_w8a8_linear_static", 16, 2, 1 << 62, 1 << 62, 32, 48, None, 64, 80, 64, 0, None)
    with pytest.raises(RuntimeError, match="2 GiB"):
        _lib.call("wf_w8a8_linear_static", 16, 1, 1 << 24, 1 << 24, 32, 48, None, (1 << 62), 80, 1 << 62, 0, None)
