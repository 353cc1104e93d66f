"""The kernels against the vendor-library routines the reference calls, run on the same GPU and data.

* The per-tensor e4m3 GEMM against torch._scaled_mm (hipBLASLt here; the reference's own call at
  wave_rt/runtime/fp8.py:49-56) on the same codes, scales and bias: within the 1e-2 relative bar of the
  W8A8 GEMM; the share of bit-equal outputs is printed.
* The int8 GEMM's int32 accumulators against torch._int_mm (hipBLASLt): bit-exact, integer arithmetic.
* The paged FP8 attention (exact form) against torch's fused bf16 attention (scaled_dot_product_attention
  restricted to its flash backend; the unfused math path is never run) over the pages the unpack kernel
  returns, the reference's non-Sage attention after its gather-dequant: max |out - sdpa| <= 2e-2, all rows.
* The dense text cross-attention against the same attention on the text keys.

A routine this torch build does not provide on this GPU skips its case with the error text.
"""

import pytest
import torch

from waveforcing_amd import _lib, inputs
from waveforcing_amd.backend import attn_dense_bf16, attn_paged_fp8
from waveforcing_amd.fp8 import _quant_rows_i8, fp8_quant_pertensor, gemm_fp8_pertensor, gemm_i8
from waveforcing_amd.kv import Fp8PagePool, PagedKV

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL_ATTN = 2e-2
TOL_GEMM = 1e-2


def _library(fn):
    try:
        out = fn()
        torch.cuda.synchronize()
        return out
    except (RuntimeError, NotImplementedError) as e:
        pytest.skip(f"torch routine unavailable here: {type(e).__name__}: {str(e).splitlines()[0][:200]}")


def _flash_sdpa(q, k, v):
    """torch's fused attention of [L, H, D] tensors, flash backend only (errors instead of falling back)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    qh, kh, vh = (t.transpose(0, 1).unsqueeze(0).contiguous() for t in (q, k, v))

    def run():
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            return torch.nn.functional.scaled_dot_product_attention(qh, kh, vh)

    return _library(run)[0].transpose(0, 1).float()


@pytest.mark.parametrize("M,N,K", [(4680, 1536, 1536), (4680, 8960, 1536), (4680, 1536, 8960), (300, 256, 1552)])
def test_fp8_gemm_against_torch_scaled_mm(M, N, K):
    seed = M + N + K
    x = inputs.outlier_activations(M, K, seed=seed, chan_seed=seed + 1).to(DEV)
    w, b = inputs.linear_weights(N, K, w_seed=seed + 2, b_seed=seed + 3)
    w, b = w.to(DEV), b.to(DEV)
    xc, xs = fp8_quant_pertensor(x, _lib.FP8_TENSOR_ACT)
    wc, ws = fp8_quant_pertensor(w, _lib.FP8_TENSOR_WEIGHT)
    y = gemm_fp8_pertensor(xc, wc, xs, ws, b)
    ref = _library(lambda: torch._scaled_mm(xc, wc.t(), scale_a=xs, scale_b=ws, bias=b, out_dtype=torch.bfloat16))
    rel = float((y.float() - ref.float()).norm() / ref.float().norm())
    equal = float((y.view(torch.int16) == ref.view(torch.int16)).float().mean())
    print(f"{M}x{N}x{K}: rel {rel:.3e}, bit-equal share {equal:.6f}")
    assert rel < TOL_GEMM, rel


@pytest.mark.parametrize("M,N,K", [(4680, 1536, 1536), (4680, 1536, 8960), (64, 256, 512)])
def test_i8_accumulators_equal_torch_int_mm(M, N, K):
    seed = 3 * M + N + K
    x = inputs.outlier_activations(M, K, seed=seed, chan_seed=seed + 1).to(DEV)
    w, b = inputs.linear_weights(N, K, w_seed=seed + 2, b_seed=seed + 3)
    qx, sx = _quant_rows_i8(x)
    qw, sw = _quant_rows_i8(w.to(DEV))
    acc = torch.empty((M, N), dtype=torch.int32, device=DEV)
    gemm_i8(qx, qw, sx, sw, b.to(DEV), acc_out=acc)
    ref = _library(lambda: torch._int_mm(qx, qw.t()))
    assert torch.equal(acc, ref)


@pytest.mark.parametrize("n_chunks,H", [(8, 12), (2, 40)])
def test_paged_attention_against_torch_flash(n_chunks, H):
    """Q [4680, H, 128] over n_chunks x 4680 keys of FP8 pages (1560-token pages at shuffled pool slots)."""
    n_kv = 4680 * n_chunks
    pages = n_kv // 1560
    pool = Fp8PagePool(2 * pages, H, 128, 1560, DEV)
    table = pool.page_table(inputs.page_table(pages, 2 * pages, seed=70 + H))
    g = torch.Generator().manual_seed(71 + H)
    k = torch.randn((n_kv, H, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((n_kv, H, 128), generator=g).to(torch.bfloat16)
    q = torch.randn((4680, H, 128), generator=g).to(torch.bfloat16).to(DEV)
    pool.pack(k.to(DEV), v.to(DEV), table)
    del k, v
    kd, vd = pool.unpack(table, n_kv)
    ref = _flash_sdpa(q, kd, vd)
    del kd, vd
    out = attn_paged_fp8(q, PagedKV(pool, table, n_kv)).float()
    err = float((out - ref).abs().max())
    print(f"{n_kv} keys, H={H}: max |out - flash sdpa| {err:.3e}")
    assert err <= TOL_ATTN, err


def test_dense_cross_attention_against_torch_flash():
    g = torch.Generator().manual_seed(80)
    q, k, v = (torch.randn((n, 12, 128), generator=g).to(torch.bfloat16).to(DEV) for n in (4680, 512, 512))
    ref = _flash_sdpa(q, k, v)
    out = attn_dense_bf16(q, k, v).float()
    err = float((out - ref).abs().max())
    print(f"dense 4680 x 512: max |out - flash sdpa| {err:.3e}")
    assert err <= TOL_ATTN, err
