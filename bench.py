"""Benchmark of the quantized DiT-block path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Headline workload: FP8 e4m3fn KV pack of 30 layers of the Wan-1.3B chunk
(K and V bf16 [4680, 12, 128] per layer, heavy-tailed, per-(token, head)
scales, 1560-token pages at seeded random page-table slots).  One step packs
all 30 layers in one kernel launch (1.307 GB of algorithmic traffic); inputs
are resident in HBM before the timed region.  The per-layer-launch rate (one
43.6 MB launch per layer, as the exchange publishes layer by layer) is
reported beside it in ``extra``.
``value`` is the algorithmic GB/s of the pack (bytes read + bytes written per
the format: 2 B in, 1 B + 4/128 B out per element).  Secondary measurements
(gather-dequant, ...) ride in ``extra``.

Prints ONE JSON line.  Only one GPU is used; --gpus above 1 exits with a
message.  The CPU baseline is the oracle's torch-CPU pack timed on a bounded
sample on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from waveforcing_amd import inputs  # noqa: E402
from waveforcing_amd.kv import Fp8PagePool  # noqa: E402

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
LAYERS, TOKENS, HEADS, HEAD_DIM, PAGE = 30, 4680, 12, 128, 1560


def profiled_traffic(name: str):
    """HBM bytes per launch recorded by the PMC runs summarized in profiles/<name>.md, or None."""
    path = os.path.join(ROOT, "profiles", name + ".md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1].split()[0]))
    return None


def kv_bytes_per_layer() -> int:
    """Algorithmic bytes of packing (or unpacking) one layer's K and V."""
    elems = TOKENS * HEADS * HEAD_DIM
    rows = TOKENS * HEADS
    return 2 * (elems * 2 + elems * 1 + rows * 4)


def _timed(fn, steps: int, warmup: int, min_warm_s: float = 0.0) -> float:
    """Mean ms per call of ``fn`` over ``steps`` calls, bracketed by HIP events on the current stream.

    Untimed warm-up: ``warmup`` calls, continued until ``min_warm_s`` seconds have passed
    (clocks of an idle GPU take a while to settle under sustained load)."""
    t0 = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t0 < min_warm_s:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


WARM_SECONDS = 1.0  # --warm-seconds


def bench_kv(steps: int, warmup: int, dev: str, which=("pack", "unpack", "pack_layers", "unpack_layers")):
    """Pack / gather-dequant of 30 layers: one launch over all layers (the
    headline) and one launch per layer (the exchange's per-layer publish)."""
    ppl = TOKENS // PAGE
    pool_pages = 2 * LAYERS * ppl
    ids = inputs.page_table(LAYERS * ppl, pool_pages, seed=7)
    pool = Fp8PagePool(pool_pages, HEADS, HEAD_DIM, PAGE, dev)
    table_all = pool.page_table(ids)
    tables = [pool.page_table(ids[i * ppl:(i + 1) * ppl]) for i in range(LAYERS)]
    k_all = torch.empty((LAYERS * TOKENS, HEADS, HEAD_DIM), dtype=torch.bfloat16, device=dev)
    v_all = torch.empty_like(k_all)
    for layer in range(LAYERS):
        k, v = inputs.kv_layer(layer)
        k_all[layer * TOKENS:(layer + 1) * TOKENS] = k.to(dev)
        v_all[layer * TOKENS:(layer + 1) * TOKENS] = v.to(dev)
    ko_all = torch.empty_like(k_all)
    vo_all = torch.empty_like(k_all)
    n_all = LAYERS * TOKENS

    def pack_all():
        pool.pack(k_all, v_all, table_all)

    def unpack_all():
        pool.unpack(table_all, n_all, out_k=ko_all, out_v=vo_all)

    def pack_layers():
        for layer in range(LAYERS):
            sl = slice(layer * TOKENS, (layer + 1) * TOKENS)
            pool.pack(k_all[sl], v_all[sl], tables[layer])

    def unpack_layers():
        for layer in range(LAYERS):
            sl = slice(layer * TOKENS, (layer + 1) * TOKENS)
            pool.unpack(tables[layer], TOKENS, out_k=ko_all[sl], out_v=vo_all[sl])

    step_bytes = LAYERS * kv_bytes_per_layer()
    fns = {"pack": pack_all, "unpack": unpack_all, "pack_layers": pack_layers, "unpack_layers": unpack_layers}
    ms = {name: _timed(fns[name], steps, warmup, min_warm_s=WARM_SECONDS) for name in which}
    out = {"bytes_per_step": step_bytes}
    for name, t in ms.items():
        out[f"ms_{name}"] = t
        out[f"{name}_gbs"] = step_bytes / (t * 1e-3) / 1e9
    return out


def bench_kv_pertensor(steps: int, warmup: int, dev: str):
    """The reference's per-tensor FP8 KV mode on one 1.3B layer: K/V [2, 4680, 12, 128] bf16 quantized with one
    scale (amax pass + quantize) and dequantized to fp32, as ``_all_gather_fp8`` does on one rank."""
    from waveforcing_amd.kv import pack_pertensor, unpack_pertensor

    k, v = inputs.kv_layer(0)
    kv = torch.stack([k, v]).to(dev)
    ms = _timed(lambda: unpack_pertensor(*pack_pertensor(kv)), steps, warmup)
    elems = kv.numel()
    moved = elems * 2 * 2 + elems * 1 + elems * 1 + elems * 4   # amax read, quant read + write, dequant read + write
    return {"us_round_trip": ms * 1e3, "bytes": moved, "gbs": moved / (ms * 1e-3) / 1e9}


def bench_gemm(steps: int, warmup: int, dev: str):
    """W8A8 linear at the Wan-1.3B shape: the int8 GEMM alone, quant + GEMM, and the
    reference's per-tensor e4m3 GEMM alone and with its activation quantization."""
    from waveforcing_amd.fp8 import WaveFp8Linear, WaveW8A8Linear, _quant_rows_i8, gemm_fp8_pertensor, gemm_i8

    x, w, b = inputs.linear_1p3b()
    x, w, b = x.to(dev), w.to(dev), b.to(dev)
    lin = WaveW8A8Linear(w, b)
    qx, sx = _quant_rows_i8(x)
    y = torch.empty((x.shape[0], w.shape[0]), dtype=torch.bfloat16, device=dev)
    reps = 50
    ms_gemm = _timed(lambda: [gemm_i8(qx, lin.w_i8, sx, lin.w_scale, lin.bias, out=y) for _ in range(reps)],
                     steps, warmup) / reps
    ms_lin = _timed(lambda: [lin(x) for _ in range(reps)], steps, warmup) / reps
    f8 = WaveFp8Linear(w, b)
    from waveforcing_amd import _lib
    from waveforcing_amd.fp8 import fp8_quant_pertensor

    xc, xs = fp8_quant_pertensor(x, _lib.FP8_TENSOR_ACT)
    ms_f8 = _timed(lambda: [gemm_fp8_pertensor(xc, f8.w_fp8, xs, f8.w_scale, f8.bias, out=y) for _ in range(reps)],
                   steps, warmup) / reps
    ms_f8_lin = _timed(lambda: [f8(x) for _ in range(reps)], steps, warmup) / reps
    M, K = x.shape
    N = w.shape[0]
    ops = 2.0 * M * N * K
    return {"ms_gemm": ms_gemm, "ms_linear": ms_lin, "ops": ops,
            "tops_gemm": ops / (ms_gemm * 1e-3) / 1e12, "tops_linear": ops / (ms_lin * 1e-3) / 1e12,
            "ms_fp8_gemm": ms_f8, "tops_fp8_gemm": ops / (ms_f8 * 1e-3) / 1e12,
            "ms_fp8_linear": ms_f8_lin, "tops_fp8_linear": ops / (ms_f8_lin * 1e-3) / 1e12}


def bench_gemm_data(steps: int, warmup: int, dev: str):
    """The int8 GEMM with uniform random int8 operands, and with A or W all zero (the same instructions, addresses
    and bytes), each timed after a second of sustained launches, at the 1.3B linear, 14B fc_out and 14B QKV
    shapes: the clock under this load depends on the operand values."""
    from waveforcing_amd.fp8 import gemm_i8

    g = torch.Generator().manual_seed(1)
    res = {}
    for name, M, N, K in (("1p3b_linear", TOKENS, 1536, 1536), ("14b_fc_out", TOKENS, 5120, 13824),
                          ("14b_qkv", TOKENS, 15360, 5120)):
        a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
        w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
        sx = (torch.rand(M, generator=g) * 0.01).to(dev)
        sw = (torch.rand(N, generator=g) * 0.01).to(dev)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        reps = 20 if K < 5000 else 5
        for tag, aa, ww in (("rand", a, w), ("zero_a", torch.zeros_like(a), w), ("zero_w", a, torch.zeros_like(w))):
            ms = _timed(lambda: [gemm_i8(aa, ww, sx, sw, None, out=y) for _ in range(reps)], steps, warmup, 1.0) / reps
            res[f"{name}_{tag}_us"] = round(ms * 1e3, 2)
            res[f"{name}_{tag}_tops"] = round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1)
        del a, w, y
    return res


def _library_call(fn, steps: int, warmup: int, reps: int, own: bool = False):
    """ms per call of a vendor-library routine, or the error text when this torch build cannot run it here
    (``own``: this library's kernel, whose errors propagate)."""
    if own:
        return _timed(lambda: [fn() for _ in range(reps)], steps, warmup) / reps, None
    try:
        fn()
        torch.cuda.synchronize()
    except (RuntimeError, NotImplementedError) as e:
        return None, f"{type(e).__name__}: {str(e).splitlines()[0][:160]}"
    return _timed(lambda: [fn() for _ in range(reps)], steps, warmup) / reps, None


def bench_library(steps: int, warmup: int, dev: str):
    """Vendor-library counterparts of the hot kernels on the same GPU, shapes and data, each beside this
    library's kernel timed in the same way:

    * torch._int_mm (hipBLASLt int8 x int8 -> int32, no scales) against the W8A8 GEMM with its fused
      dequant + bias epilogue at the 1.3B linear 4680 x 1536 x 1536;
    * the reference's per-tensor e4m3 linear as it calls it, torch._scaled_mm(x_fp8, w_fp8.t(), s_x, s_w,
      bias, bf16) (wave_rt/runtime/fp8.py:49-56), against wf_gemm_fp8_pertensor on the same codes;
    * torch's fused bf16 attention (scaled_dot_product_attention restricted to its flash and
      memory-efficient backends; the unfused math path is never used) over the dequantized pages, the
      reference's non-Sage attention after its gather-dequant, against the paged FP8 kernel's three forms
      on the same pages (Q [4680, 12, 128] over 37440 keys)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from waveforcing_amd.backend import attn_paged_fp8
    from waveforcing_amd.fp8 import (WaveFp8Linear, WaveW8A8Linear, _quant_rows_i8, gemm_fp8_pertensor,
                                     gemm_i8)
    from waveforcing_amd.kv import PagedKV

    res = {}
    x, w, b = inputs.linear_1p3b()
    x, w, b = x.to(dev), w.to(dev), b.to(dev)
    M, K = x.shape
    N = w.shape[0]
    ops = 2.0 * M * N * K
    lin = WaveW8A8Linear(w, b)
    qx, sx = _quant_rows_i8(x)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    wt = lin.w_i8.t()
    reps = 50
    for name, fn in (("w8a8_gemm", lambda: gemm_i8(qx, lin.w_i8, sx, lin.w_scale, lin.bias, out=y)),
                     ("torch_int_mm", lambda: torch._int_mm(qx, wt))):
        ms, err = _library_call(fn, steps, warmup, reps, own=name == "w8a8_gemm")
        res[f"{name}_us"] = None if ms is None else round(ms * 1e3, 2)
        res[f"{name}_tops"] = None if ms is None else round(ops / (ms * 1e-3) / 1e12, 1)
        if err:
            res[f"{name}_error"] = err
    f8 = WaveFp8Linear(w, b)
    from waveforcing_amd import _lib
    from waveforcing_amd.fp8 import fp8_quant_pertensor

    xc, xs = fp8_quant_pertensor(x, _lib.FP8_TENSOR_ACT)
    w8t = f8.w_fp8.t()
    for name, fn in (("fp8_gemm", lambda: gemm_fp8_pertensor(xc, f8.w_fp8, xs, f8.w_scale, f8.bias, out=y)),
                     ("torch_scaled_mm", lambda: torch._scaled_mm(xc, w8t, scale_a=xs, scale_b=f8.w_scale,
                                                                   bias=f8.bias, out_dtype=torch.bfloat16))):
        ms, err = _library_call(fn, steps, warmup, reps, own=name == "fp8_gemm")
        res[f"{name}_us"] = None if ms is None else round(ms * 1e3, 2)
        res[f"{name}_tflops"] = None if ms is None else round(ops / (ms * 1e-3) / 1e12, 1)
        if err:
            res[f"{name}_error"] = err
    # the 14B fc_out, 4680 x 5120 x 13824 (long K), on N(0, 1) activations and weights drawn on the GPU
    gen = torch.Generator(device=dev).manual_seed(5)
    M2, N2, K2 = TOKENS, 5120, 13824
    ops2 = 2.0 * M2 * N2 * K2
    x2 = torch.randn((M2, K2), generator=gen, device=dev).to(torch.bfloat16)
    w2 = (torch.randn((N2, K2), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    y2 = torch.empty((M2, N2), dtype=torch.bfloat16, device=dev)
    qx2, sx2 = _quant_rows_i8(x2)
    qw2, sw2 = _quant_rows_i8(w2)
    xc2, xs2 = fp8_quant_pertensor(x2, _lib.FP8_TENSOR_ACT)
    wc2, ws2 = fp8_quant_pertensor(w2, _lib.FP8_TENSOR_WEIGHT)
    del x2, w2
    qw2t, wc2t = qw2.t(), wc2.t()
    for name, fn, unit in (
            ("14b_fc_out_w8a8_gemm", lambda: gemm_i8(qx2, qw2, sx2, sw2, None, out=y2), "tops"),
            ("14b_fc_out_torch_int_mm", lambda: torch._int_mm(qx2, qw2t), "tops"),
            ("14b_fc_out_fp8_gemm", lambda: gemm_fp8_pertensor(xc2, wc2, xs2, ws2, None, out=y2), "tflops"),
            ("14b_fc_out_torch_scaled_mm", lambda: torch._scaled_mm(xc2, wc2t, scale_a=xs2, scale_b=ws2,
                                                                     out_dtype=torch.bfloat16), "tflops")):
        ms, err = _library_call(fn, steps, warmup, 3, own="torch" not in name)
        res[f"{name}_us"] = None if ms is None else round(ms * 1e3, 2)
        res[f"{name}_{unit}"] = None if ms is None else round(ops2 / (ms * 1e-3) / 1e12, 1)
        if err:
            res[f"{name}_error"] = err
    del qx2, qw2, xc2, wc2, y2
    if res.get("torch_scaled_mm_us") is not None:
        ref = torch._scaled_mm(xc, w8t, scale_a=xs, scale_b=f8.w_scale, bias=f8.bias, out_dtype=torch.bfloat16)
        mine = gemm_fp8_pertensor(xc, f8.w_fp8, xs, f8.w_scale, f8.bias)
        res["fp8_gemm_vs_torch_scaled_mm_max_rel"] = float(
            ((mine.float() - ref.float()).abs().max() / ref.float().abs().max()).item())
    del x, w, y, qx, xc, lin, f8

    H = HEADS
    n_kv = TOKENS * 8
    pages = n_kv // PAGE
    pool = Fp8PagePool(2 * pages, H, HEAD_DIM, PAGE, dev)
    table = pool.page_table(inputs.page_table(pages, 2 * pages, seed=11))
    g = torch.Generator().manual_seed(12)
    k = torch.randn((n_kv, H, HEAD_DIM), generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn((n_kv, H, HEAD_DIM), generator=g).to(torch.bfloat16).to(dev)
    pool.pack(k, v, table)
    del k, v
    q = torch.randn((TOKENS, H, HEAD_DIM), generator=g).to(torch.bfloat16).to(dev)
    ctx = PagedKV(pool, table, n_kv)
    out = torch.empty_like(q)
    flops = 4.0 * TOKENS * n_kv * H * HEAD_DIM
    for form, kw in ATTN_FORMS.items():
        ms, _ = _library_call(lambda: attn_paged_fp8(q, ctx, out=out, **kw), steps, warmup, 1, own=True)
        res[f"attn_paged_fp8_{form}_ms"] = round(ms, 4)
    kd, vd = pool.unpack(table, n_kv)
    qh = q.transpose(0, 1).unsqueeze(0).contiguous()
    kh = kd.transpose(0, 1).unsqueeze(0).contiguous()
    vh = vd.transpose(0, 1).unsqueeze(0).contiguous()
    del kd, vd
    for name, backend in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        def sdpa(backend=backend):
            with sdpa_kernel([backend]):
                return torch.nn.functional.scaled_dot_product_attention(qh, kh, vh)
        ms, err = _library_call(sdpa, steps, warmup, 1)
        res[f"torch_sdpa_{name}_ms"] = None if ms is None else round(ms, 4)
        if ms is not None:
            res[f"torch_sdpa_{name}_tflops"] = round(flops / (ms * 1e-3) / 1e12, 1)
            o_ref = sdpa()[0].transpose(0, 1).float()
            attn_paged_fp8(q, ctx, out=out)
            torch.cuda.synchronize()
            res[f"attn_bf16_vs_torch_sdpa_{name}_max_abs"] = float((out.float() - o_ref).abs().max().item())
        if err:
            res[f"torch_sdpa_{name}_error"] = err
    res["note"] = ("vendor-library routines on the same GPU and data: torch._int_mm (hipBLASLt, int32 out, no "
                   "epilogue) and the reference's torch._scaled_mm e4m3 linear at 4680x1536x1536 and at the 14B "
                   "fc_out 4680x5120x13824 (no bias there); torch's fused "
                   "bf16 SDPA (flash / memory-efficient backends only) over the unpacked pages at 4680 queries x "
                   "37440 keys x 12 heads, beside this library's kernels")
    return res


def bench_block_linears(steps: int, warmup: int, dev: str):
    """The Wan-1.3B block's W8A8 GEMMs on one 4680-token chunk as the block runs them: fused QKV [4608, 1536],
    O [1536, 1536], fc_in [8960, 1536], fc_out [1536, 8960] (activations pre-quantized; 345.97 G int8 ops per
    step; the FFN's GELU runs in fc_out's input quantizer, outside these GEMMs)."""
    from waveforcing_amd.fp8 import _quant_rows_i8, gemm_i8

    M = TOKENS
    shapes = [(4608, 1536, False), (1536, 1536, False), (8960, 1536, False), (1536, 8960, False)]
    ops = 0.0
    calls = []
    for i, (N, K, gelu) in enumerate(shapes):
        x = inputs.outlier_activations(M, K, seed=20 + i, chan_seed=30 + i).to(dev)
        w, b = inputs.linear_weights(N, K, w_seed=40 + i, b_seed=50 + i)
        qx, sx = _quant_rows_i8(x)
        qw, sw = _quant_rows_i8(w.to(dev))
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        calls.append((qx, qw, sx, sw, b.to(dev), gelu, y))
        ops += 2.0 * M * N * K

    def step():
        for qx, qw, sx, sw, b, gelu, y in calls:
            gemm_i8(qx, qw, sx, sw, b, gelu=gelu, out=y)

    ms = _timed(step, steps, warmup)
    return {"ms": ms, "ops": ops, "tops": ops / (ms * 1e-3) / 1e12}


ATTN_FORMS = {"bf16": {}, "qk8": {"quantized_qk": True}, "qkpv8": {"fp8_pv": True}}


def bench_attention(steps: int, warmup: int, dev: str, chunks: int = 8, form: str = "bf16",
                    zero_k: bool = False, zero_v: bool = False, warm_s: float = 0.0):
    """Paged FP8 attention: Q [4680, 12, 128] over `chunks` chunks (4680 keys each) of FP8 pages.  ``form``:
    "bf16" the exact form, "qk8" e4m3 queries against the K codes on the fp8 matrix cores, "qkpv8" that and
    e4m3 weights against the V codes.  ``zero_k`` / ``zero_v`` pack zeros in place of the N(0, 1) K / V (the
    same addresses and work)."""
    from waveforcing_amd.backend import attn_paged_fp8
    from waveforcing_amd.kv import PagedKV

    H = HEADS
    n_kv = TOKENS * chunks
    pages = n_kv // PAGE
    pool = Fp8PagePool(2 * pages, H, HEAD_DIM, PAGE, dev)
    table = pool.page_table(inputs.page_table(pages, 2 * pages, seed=11))
    g = torch.Generator().manual_seed(12)
    k = torch.randn((n_kv, H, HEAD_DIM), generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn((n_kv, H, HEAD_DIM), generator=g).to(torch.bfloat16).to(dev)
    pool.pack(torch.zeros_like(k) if zero_k else k, torch.zeros_like(v) if zero_v else v, table)
    del k, v
    q = torch.randn((TOKENS, H, HEAD_DIM), generator=g).to(torch.bfloat16).to(dev)
    ctx = PagedKV(pool, table, n_kv)
    out = torch.empty_like(q)
    kw = ATTN_FORMS[form]
    ms = _timed(lambda: attn_paged_fp8(q, ctx, out=out, **kw), steps, warmup, warm_s)
    flops = 4.0 * TOKENS * n_kv * H * HEAD_DIM
    return {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "flops": flops, "keys": n_kv}


def bench_attention_data(steps: int, warmup: int, dev: str, repeats: int = 2):
    """The three attention forms on the attention workload with N(0, 1) or zero K / V in the pages, each timed
    after a second of sustained launches: the clock under this load depends on the operand values."""
    res = {}
    for rep in range(repeats):
        for name, zk, zv in (("randn", False, False), ("zero", True, True), ("zero_k", True, False),
                             ("zero_v", False, True)):
            for form in ATTN_FORMS:
                r = bench_attention(steps, warmup, dev, form=form, zero_k=zk, zero_v=zv, warm_s=1.0)
                res[f"{name}{'' if form == 'bf16' else '_' + form}_ms_{rep}"] = round(r["ms"], 4)
    return res


def bench_block(scale: str, steps: int, warmup: int, dev: str, form: str = "bf16"):
    """One quantized DiT block over one 3-frame chunk (4680 tokens, 30x52 latent grid) with 7 prior
    chunks of FP8 paged context (37440 keys incl. its own) and a 512-token text context; ``form`` selects
    the self-attention backend (bf16: hip_fp8, qk8: hip_fp8_qk, qkpv8: hip_fp8_qkpv)."""
    from waveforcing_amd import rope
    from waveforcing_amd.backend import _WAVE_STATE, enable_hip_fp8, enable_hip_fp8_qk, enable_hip_fp8_qkpv
    from waveforcing_amd.block import PRESETS, QuantizedWanBlock, random_block_params

    cfg = PRESETS[scale]
    dim, heads, ffn = cfg["dim"], cfg["heads"], cfg["ffn_dim"]
    frames, h, w = 3, 30, 52
    T = frames * h * w
    prior = 7
    pages = (prior + 1) * frames
    blk = QuantizedWanBlock(random_block_params(dim, ffn, seed=3), heads, dev)
    pool = Fp8PagePool(pages, heads, HEAD_DIM, PAGE, dev)
    g = torch.Generator().manual_seed(4)
    prior_kv = torch.randn((prior * T, heads, HEAD_DIM), generator=g).to(torch.bfloat16).to(dev)
    pool.pack(prior_kv, prior_kv, pool.page_table(list(range(prior * frames))))
    del prior_kv
    ctx = pool.page_table(list(range(pages)))
    own = pool.page_table(list(range(prior * frames, pages)))
    text = torch.randn((512, dim), generator=g).to(torch.bfloat16).to(dev)
    tkv = blk.text_kv(text)
    cos, sin = rope.cos_sin(frames, h, w, prior * frames, device=dev)
    x0 = torch.randn((T, dim), generator=g).to(torch.bfloat16).to(dev)
    e = (torch.randn((frames, 6, dim), generator=g) * 0.1).to(torch.bfloat16).to(dev)
    x = x0.clone()

    def step():
        x.copy_(x0)
        blk.forward(x, e, cos, sin, pool, ctx, own, (prior + 1) * T, tkv)

    saved = dict(_WAVE_STATE)
    try:
        {"bf16": enable_hip_fp8, "qk8": enable_hip_fp8_qk, "qkpv8": enable_hip_fp8_qkpv}[form]()
        ms = _timed(step, steps, warmup)
    finally:
        _WAVE_STATE.clear()
        _WAVE_STATE.update(saved)
    return {"ms": ms, "tokens": T, "context_keys": (prior + 1) * T}


def _prefill_clean(x, filler, n_clean: int = 8) -> None:
    """Fill every layer's clean list of exchange ``x`` with ``n_clean`` chunks of ``filler`` K/V (slots packed
    directly), the first one the anchor with ``filler`` as its un-rotated K."""
    from waveforcing_amd.exchange import CleanPage

    for layer in range(x.n_layers):
        for cid in range(n_clean):
            slot = x.reserve(layer)
            x.pack(layer, slot, filler, filler)
            x.append_clean(layer, CleanPage(cid, slot))
    x.anchor_ku = filler.unsqueeze(0).expand(x.n_layers, *filler.shape).contiguous()


STEADY_TICK = 12  # rf_step 4 with 8 clean chunks (0..7): the store rank stores chunk 8, ranks 0..3 hold 12..9


def bench_exchange(steps: int, warmup: int, dev: str):
    """The paged exchange of one steady-state wavefront tick over the 30 Wan-1.3B layers (rf_step 4, 21-frame
    window, clean list anchor + 7): the store pass and the four denoise passes each pack their chunk's K/V into
    its slot per layer, and the anchor's K is re-RoPEd for the store geometry and for the denoise geometry (one
    launch over all layers each).  Rank 0's context is anchor + 2 working + live + self + 3 in-flight = 37440
    keys."""
    from waveforcing_amd.exchange import PagedExchange, TickPlan

    x = PagedExchange(LAYERS, HEADS, PAGE, frames_per_chunk=3, max_attn_frames=21, rf_step=4, device=dev)
    g = torch.Generator().manual_seed(21)
    filler = torch.randn((TOKENS, HEADS, HEAD_DIM), generator=g).to(torch.bfloat16).to(dev)
    _prefill_clean(x, filler)
    k, v = inputs.kv_layer(0)
    k, v = k.to(dev).unsqueeze(0), v.to(dev).unsqueeze(0)
    plan = TickPlan(STEADY_TICK, [0, 1, 2, 3], True, (STEADY_TICK - 3) * 3, 12)
    n_ctx = []

    def step():
        x.begin_tick(plan)
        for exch in [x.make_store_exch()] + [x.make_denoise_exch(r) for r in (3, 2, 1, 0)]:
            for layer in range(LAYERS):
                ctx, _ = exch(layer_idx=layer, roped_query=None, roped_key=k, unroped_key=None, value=v,
                              post_patch_height=30, post_patch_width=52)
        n_ctx.append(ctx.n_tokens)
        x.abort_tick()   # keep the clean lists as they are: every timed tick is the same steady-state tick

    ms = _timed(step, steps, warmup)
    elems = TOKENS * HEADS * HEAD_DIM
    rows = TOKENS * HEADS
    anchor_bytes = LAYERS * (elems * 2 + elems + rows * 4)   # K only: read bf16, write codes + scales
    tick_bytes = 5 * LAYERS * kv_bytes_per_layer() + 2 * anchor_bytes
    return {"ms_per_tick": ms, "us_per_pass_layer": ms * 1e3 / (5 * LAYERS), "bytes_per_tick": tick_bytes,
            "gbs": tick_bytes / (ms * 1e-3) / 1e9, "rank0_context_keys": n_ctx[-1]}


def bench_stack(steps: int, warmup: int, dev: str, preset: str = "1.3b", ticks_only: bool = False):
    """A steady-state wavefront tick of all the Wan blocks of a preset (30 for 1.3B, 40 for 14B) on one GPU:
    rf_step 4, 21-frame window, 3-frame chunks of 4680 tokens (30x52 grid), 512-token text context.  8 store
    passes through the stack fill the clean list (anchor + 7); the timed tick is tick 12: the store pass of
    chunk 8 and the denoise passes of ranks 3..0 (chunks 9..12), each with its anchor re-RoPE and fused in-block
    K/V pack.  Rank 0's pass -- one denoise step of one chunk -- attends over anchor + 2 working + live + self +
    3 in-flight = 37440 keys and is also timed alone."""
    from waveforcing_amd.exchange import TickPlan
    from waveforcing_amd.stack import QuantizedWanStack

    frames, h, w = 3, 30, 52
    st = QuantizedWanStack.random(preset, seed=100, device=dev, tokens_per_frame=h * w, frames_per_chunk=frames,
                                  max_attn_frames=21, rf_step=4)
    ex = st.exchange
    dim = st.blocks[0].dim
    g = torch.Generator(device=dev).manual_seed(5)
    st.set_text(torch.randn((512, dim), generator=g, device=dev).to(torch.bfloat16))
    T = frames * h * w
    x0 = torch.randn((T, dim), generator=g, device=dev).to(torch.bfloat16)
    e = (torch.randn((frames, 6, dim), generator=g, device=dev) * 0.1).to(torch.bfloat16)
    xs = {k: x0.clone() for k in ("store", 0, 1, 2, 3)}
    for c in range(8):
        xs["store"].copy_(x0)
        st.forward_chunk(xs["store"], e, c, h, w, store=True)
    plan = TickPlan(STEADY_TICK, [0, 1, 2, 3], True, (STEADY_TICK - 3) * frames, 4 * frames)

    def tick():
        ex.begin_tick(plan)
        try:
            for key in ("store", 3, 2, 1, 0):
                xs[key].copy_(x0)
                p = ex.store_pass() if key == "store" else ex.denoise_pass(key)
                st.run_pass(xs[key], e, p, h, w)
        finally:
            ex.abort_tick()   # the clean lists stay as they are: every timed tick is the same

    ms_tick = _timed(tick, max(2, steps // 3), 1)

    def tick_concurrent():
        ex.begin_tick(plan)
        try:
            for key in ("store", 3, 2, 1, 0):
                xs[key].copy_(x0)
            st.run_pass(xs["store"], e, ex.store_pass(), h, w)
            st.run_wavefront([(xs[r], e, ex.denoise_pass(r)) for r in (3, 2, 1, 0)], h, w)
        finally:
            ex.abort_tick()

    ms_tick_con = _timed(tick_concurrent, max(2, steps // 3), 1)
    if ticks_only:
        out = {"ms_per_tick_5_passes": ms_tick, "ms_per_tick_5_passes_concurrent": ms_tick_con}
        del st, xs, x0
        torch.cuda.empty_cache()
        return out
    # rank 0's pass alone, inside an open tick whose other passes have run
    ex.begin_tick(plan)
    for key in ("store", 3, 2, 1):
        p = ex.store_pass() if key == "store" else ex.denoise_pass(key)
        st.run_pass(xs[key], e, p, h, w)
    p0 = ex.denoise_pass(0)
    n_ctx = ex.layer_context(0, p0, h, w)[3]

    def step():
        xs[0].copy_(x0)
        st.run_pass(xs[0], e, p0, h, w)

    ms = _timed(step, steps, warmup)
    ex.abort_tick()
    out = {"ms": ms, "ms_per_layer": ms / len(st.blocks), "layers": len(st.blocks), "tokens": T,
           "context_keys": n_ctx, "tokens_per_s": T / (ms * 1e-3), "ms_per_tick_5_passes": ms_tick,
           "ms_per_tick_5_passes_concurrent": ms_tick_con}
    del st, xs, x0
    torch.cuda.empty_cache()
    return out


def bench_dit(steps: int, warmup: int, dev: str, preset: str = "1.3b", form: str = "bf16"):
    """The whole DiT forward of one chunk from its noisy latent [1, 16, 3, 60, 104] to x0 (patch embedding, time
    embedding, the 30 blocks over the paged exchange, head, unpatchify and flow -> x0), as rank 0's pass of the
    same steady-state tick as bench_stack (37440-key context), at the first DMD timestep; ``form`` selects the
    self-attention backend as in bench_block."""
    from waveforcing_amd.backend import _WAVE_STATE, enable_hip_fp8, enable_hip_fp8_qk, enable_hip_fp8_qkpv
    from waveforcing_amd.dit import QuantizedWanDiT, random_dit_params
    from waveforcing_amd.exchange import TickPlan
    from waveforcing_amd.stack import QuantizedWanStack

    frames, H, W = 3, 60, 104
    st = QuantizedWanStack.random(preset, seed=100, device=dev, tokens_per_frame=(H // 2) * (W // 2),
                                  frames_per_chunk=frames, max_attn_frames=21, rf_step=4)
    ex = st.exchange
    dit = QuantizedWanDiT(random_dit_params(st.blocks[0].dim, seed=7, device=dev), st)
    g = torch.Generator(device=dev).manual_seed(6)
    dit.set_text(torch.randn((512, 4096), generator=g, device=dev).to(torch.bfloat16))
    noisy = torch.randn((1, 16, frames, H, W), generator=g, device=dev).to(torch.bfloat16)
    steps_t = dit.schedule.warp()
    for c in range(8):
        dit.forward_chunk(noisy, 0.0, chunk=c, store=True)
    plan = TickPlan(STEADY_TICK, [0, 1, 2, 3], True, (STEADY_TICK - 3) * frames, 4 * frames)
    ex.begin_tick(plan)
    dit.run_pass(noisy, 0.0, ex.store_pass(), want_x0=False)
    for r in (3, 2, 1):
        dit.run_pass(noisy, steps_t[r], ex.denoise_pass(r))
    p0 = ex.denoise_pass(0)
    x0 = torch.empty((1, frames, 16, H, W), dtype=torch.bfloat16, device=dev)

    def step():
        dit.run_pass(noisy, steps_t[0], p0, x0_out=x0)

    saved = dict(_WAVE_STATE)
    try:
        {"bf16": enable_hip_fp8, "qk8": enable_hip_fp8_qk, "qkpv8": enable_hip_fp8_qkpv}[form]()
        ms = _timed(step, steps, warmup)
    finally:
        _WAVE_STATE.clear()
        _WAVE_STATE.update(saved)
    ex.abort_tick()
    T = frames * (H // 2) * (W // 2)
    out = {"ms": ms, "layers": len(st.blocks), "tokens": T, "latent": [1, 16, frames, H, W],
           "timestep": steps_t[0], "tokens_per_s": T / (ms * 1e-3)}
    del dit, st
    torch.cuda.empty_cache()
    return out


def bench_generate(steps: int, warmup: int, dev: str, chunks: int = 12):
    """WavefrontDenoiser.generate: one stream of `chunks` 3-frame chunks from noise [1, 16, 3 chunks, 60, 104] to
    clean latents through the 30-block 1.3B DiT (rf_step 4, the four warped DMD steps, 21-frame window, 512-token
    text context): chunks + 4 ticks, each the store pass and the active denoise ranks as a layer wavefront, the
    re-noising between steps included; the exchange is reset at the start of each stream.  The ramp-up and drain
    ticks hold fewer passes than the steady state."""
    from waveforcing_amd.dit import QuantizedWanDiT, random_dit_params
    from waveforcing_amd.stack import QuantizedWanStack
    from waveforcing_amd.wavefront import WavefrontDenoiser

    frames, H, W = 3, 60, 104
    st = QuantizedWanStack.random("1.3b", seed=100, device=dev, tokens_per_frame=(H // 2) * (W // 2),
                                  frames_per_chunk=frames, max_attn_frames=21, rf_step=4)
    dit = QuantizedWanDiT(random_dit_params(st.blocks[0].dim, seed=7, device=dev), st)
    g = torch.Generator(device=dev).manual_seed(6)
    dit.set_text(torch.randn((512, 4096), generator=g, device=dev).to(torch.bfloat16))
    noise = torch.randn((1, 16, frames * chunks, H, W), generator=g, device=dev).to(torch.bfloat16)
    den = WavefrontDenoiser(dit)
    ms = _timed(lambda: den.generate(noise, concurrent=True), steps, warmup)
    ticks = chunks + den.rf_step
    out = {"ms_per_stream": ms, "chunks": chunks, "ticks": ticks, "ms_per_tick_mean": ms / ticks,
           "latent_frames_per_s": frames * chunks / (ms * 1e-3), "latent": [1, 16, frames * chunks, H, W]}
    del den, dit, st
    torch.cuda.empty_cache()
    return out


def bench_copy(steps: int, warmup: int, dev: str):
    """A plain device copy of 1 GiB (read 1 GiB + write 1 GiB): calibrates the HBM byte counters."""
    src = torch.empty((1 << 30,), dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    ms = _timed(lambda: dst.copy_(src), steps, warmup)
    return {"ms": ms, "bytes_read": 1 << 30, "bytes_written": 1 << 30, "gbs": 2 * (1 << 30) / (ms * 1e-3) / 1e9}


def _cpu_model() -> str:
    """The host CPU's model name (first ``model name`` line of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


CPU_MODEL = _cpu_model()


def cpu_baseline_kv() -> dict:
    """Oracle torch-CPU pack (quantize + page scatter) of a bounded sample of layers."""
    from oracle import kv as okv

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    ppl = TOKENS // PAGE
    n_layers = 2
    kc, kscale = okv.new_pool(n_layers * ppl, PAGE, HEADS, HEAD_DIM)
    vc, vscale = okv.new_pool(n_layers * ppl, PAGE, HEADS, HEAD_DIM)
    data = [inputs.kv_layer(i) for i in range(n_layers)]

    def run():
        for i, (k, v) in enumerate(data):
            table = list(range(i * ppl, (i + 1) * ppl))
            okv.pack(k, table, PAGE, kc, kscale)
            okv.pack(v, table, PAGE, vc, vscale)

    run()  # warm-up
    reps = []
    t_end = time.perf_counter() + 15.0
    while len(reps) < 5 or (time.perf_counter() < t_end and len(reps) < 30):
        t0 = time.perf_counter()
        run()
        reps.append(time.perf_counter() - t0)
    reps.sort()
    med = reps[len(reps) // 2]
    gbs = n_layers * kv_bytes_per_layer() / med / 1e9
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": threads, "cpu_model": CPU_MODEL,
        "kind": "port",
        "sample": f"oracle torch-CPU pack of {n_layers} of the 30 layers (K and V), median of {len(reps)} reps",
    }


def _cpu_median(fn, reps: int = 5, budget_s: float = 6.0) -> float:
    fn()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 2 or (len(times) < reps and time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def cpu_baseline_extra() -> dict:
    """The oracle's torch-CPU path of the other workloads, timed on this host: the int8 W8A8 linear at the
    1.3B shape (whole), the reference's per-tensor e4m3 linear (64 rows) and the attention over 8 chunks
    (256 queries of one head against all 37440 keys), the last two extrapolated to the full workload, and
    the whole 1.3B block."""
    from oracle import attention as oat
    from oracle import linear as olin

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    out = {}
    x, w, b = inputs.linear_1p3b()
    ops = 2.0 * x.shape[0] * w.shape[0] * x.shape[1]
    t = _cpu_median(lambda: olin.i8_linear(x, w, b))
    out["w8a8_int8_linear"] = {"value": round(ops / t / 1e12, 4), "unit": "TOPS", "ms": round(t * 1e3, 2),
                               "cores": threads, "cpu_model": CPU_MODEL, "kind": "port",
                               "sample": "oracle int8 linear 4680x1536x1536 incl. quantization (torch _int_mm)"}
    wq, ws = olin.fp8_quant_weight(w)
    rows = 64  # torch's CPU _scaled_mm is slow (~80 s for the whole 4680-row linear): a bounded sample
    t = _cpu_median(lambda: olin.fp8_linear(x[:rows], wq, ws, b), reps=3)
    ops_s = 2.0 * rows * w.shape[0] * x.shape[1]
    out["fp8_pertensor_linear"] = {"value": round(ops_s / t / 1e12, 6), "unit": "TFLOP/s",
                                   "ms_full_workload_extrapolated": round(t * x.shape[0] / rows * 1e3, 1),
                                   "cores": threads, "cpu_model": CPU_MODEL, "kind": "port",
                                   "sample": "oracle per-tensor e4m3 linear, 64 of the 4680 rows x 1536 x 1536 "
                                             "(torch _scaled_mm)"}
    g = torch.Generator().manual_seed(12)
    n_kv, lq = 8 * TOKENS, 256
    q = torch.randn((lq, 1, HEAD_DIM), generator=g).to(torch.bfloat16)
    kv = torch.randn((n_kv, 1, HEAD_DIM), generator=g).to(torch.bfloat16)
    t = _cpu_median(lambda: oat.sdpa(q, kv, kv), reps=3)
    flops = 4.0 * lq * n_kv * HEAD_DIM
    full_ms = t * (TOKENS * HEADS) / lq * 1e3
    out["attention_8_chunks"] = {"value": round(flops / t / 1e12, 4), "unit": "TFLOP/s",
                                 "ms_full_workload_extrapolated": round(full_ms, 1), "cores": threads, "cpu_model": CPU_MODEL, "kind": "port",
                                 "sample": "oracle SDPA, 256 queries x 1 head over 37440 keys, fp32; x 219.4 "
                                           "extrapolates to 4680 queries x 12 heads"}
    out["dit_block_1p3b"] = cpu_baseline_block(threads)
    return out


def cpu_baseline_block(threads: int) -> dict:
    """The oracle's CPU block (oracle.block.block_forward) on the whole 1.3B block workload: 4680 tokens,
    7 prior chunks + its own of FP8 paged context (37440 keys), 512 text tokens (text K/V outside the timing,
    as on the GPU), random init; the 30-layer stack figure is 30 x that."""
    from oracle import block as ob
    from oracle import kv as okv
    from waveforcing_amd.block import PRESETS, random_block_params

    cfg = PRESETS["1.3b"]
    dim, heads, ffn = cfg["dim"], cfg["heads"], cfg["ffn_dim"]
    frames, h, w = 3, 30, 52
    T = frames * h * w
    prior = 7
    pages = (prior + 1) * frames
    params = random_block_params(dim, ffn, seed=3)
    g = torch.Generator().manual_seed(4)
    pk = okv.new_pool(pages, PAGE, heads, HEAD_DIM)
    pv = okv.new_pool(pages, PAGE, heads, HEAD_DIM)
    prior_kv = torch.randn((prior * T, heads, HEAD_DIM), generator=g).to(torch.bfloat16)
    okv.pack(prior_kv, list(range(prior * frames)), PAGE, *pk)
    okv.pack(prior_kv, list(range(prior * frames)), PAGE, *pv)
    del prior_kv
    text = torch.randn((512, dim), generator=g).to(torch.bfloat16)
    tk, tv = ob.text_kv(params, text, heads)
    x = torch.randn((T, dim), generator=g).to(torch.bfloat16)
    e = (torch.randn((frames, 6, dim), generator=g) * 0.1).to(torch.bfloat16)
    ctx, own = list(range(pages)), list(range(prior * frames, pages))
    t = _cpu_median(lambda: ob.block_forward(params, x, e, (frames, h, w), prior * frames, pk, pv, ctx, own,
                                             (prior + 1) * T, PAGE, tk, tv, heads), reps=3, budget_s=8.0)
    return {"value": round(t * 1e3, 1), "unit": "ms per block per 3-frame chunk", "higher_is_better": False,
            "ms_30_layer_stack_extrapolated": round(30 * t * 1e3, 0), "cores": threads, "cpu_model": CPU_MODEL, "kind": "port",
            "sample": "oracle block_forward, whole 1.3B block: 4680 tokens over 37440 FP8 paged keys + 512 text "
                      "tokens (int8 _int_mm linears, fp32 SDPA)"}


def main() -> None:
    global WARM_SECONDS
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--warm-seconds", type=float, default=WARM_SECONDS,
                    help="minimum untimed warm-up of the KV workloads (profiler runs use 0)")
    ap.add_argument("--only", choices=["kv", "kv_pack", "kv_unpack", "gemm", "linears_1p3b", "attention", "cpu_extra",
                                       "block_1p3b", "block_14b", "exchange_1p3b", "stack_1p3b", "stack_14b", "dit_1p3b",
                                       "tick_1p3b", "generate_1p3b", "copy", "attention_qk8", "block_1p3b_qk8",
                                       "attention_qkpv8", "block_1p3b_qkpv8", "block_14b_qkpv8", "dit_1p3b_qkpv8",
                                       "kv_pertensor",
                                       "attention_data", "gemm_data", "library"],
                    help="run one workload alone (for profiler runs) and print its own JSON line")
    args = ap.parse_args()
    WARM_SECONDS = args.warm_seconds
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the path runs on a single GPU); --gpus {args.gpus} is not supported",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = "cuda:0"
    if args.only:
        fn = {"kv": bench_kv, "kv_pack": lambda s, w, d: bench_kv(s, w, d, ("pack",)),
              "kv_unpack": lambda s, w, d: bench_kv(s, w, d, ("unpack",)), "gemm": bench_gemm,
              "linears_1p3b": bench_block_linears, "attention": bench_attention, "copy": bench_copy,
              "block_1p3b": lambda s, w, d: bench_block("1.3b", s, w, d),
              "block_14b": lambda s, w, d: bench_block("14b", s, w, d), "exchange_1p3b": bench_exchange,
              "stack_1p3b": bench_stack, "stack_14b": lambda s, w, d: bench_stack(s, w, d, "14b"),
              "dit_1p3b": bench_dit, "tick_1p3b": lambda s, w, d: bench_stack(s, w, d, ticks_only=True),
              "generate_1p3b": bench_generate,
              "attention_qk8": lambda s, w, d: bench_attention(s, w, d, form="qk8"),
              "block_1p3b_qk8": lambda s, w, d: bench_block("1.3b", s, w, d, form="qk8"),
              "attention_qkpv8": lambda s, w, d: bench_attention(s, w, d, form="qkpv8"),
              "block_1p3b_qkpv8": lambda s, w, d: bench_block("1.3b", s, w, d, form="qkpv8"),
              "block_14b_qkpv8": lambda s, w, d: bench_block("14b", s, w, d, form="qkpv8"),
              "library": bench_library,
              "dit_1p3b_qkpv8": lambda s, w, d: bench_dit(s, w, d, form="qkpv8"),
              "kv_pertensor": bench_kv_pertensor, "attention_data": bench_attention_data,
              "gemm_data": bench_gemm_data,
              "cpu_extra": lambda s, w, d: cpu_baseline_extra()}[args.only]
        print(json.dumps({"only": args.only, **fn(args.steps, args.warmup, dev)}), flush=True)
        return
    kv = bench_kv(args.steps, args.warmup, dev)
    gm = bench_gemm(max(5, args.steps // 5), 2, dev)
    lin = bench_block_linears(max(5, args.steps // 5), 2, dev)
    at_sweep = {c: bench_attention(max(5, args.steps // 5), 2, dev, chunks=c) for c in (1, 2, 4, 8)}
    at = at_sweep[8]
    at_qk = bench_attention(max(5, args.steps // 5), 2, dev, form="qk8")
    at_pv = bench_attention(max(5, args.steps // 5), 2, dev, form="qkpv8")
    kvt = bench_kv_pertensor(max(5, args.steps // 5), 2, dev)
    b13 = bench_block("1.3b", max(5, args.steps // 5), 2, dev)
    b13q = bench_block("1.3b", max(5, args.steps // 5), 2, dev, form="qk8")
    b13p = bench_block("1.3b", max(5, args.steps // 5), 2, dev, form="qkpv8")
    b14 = bench_block("14b", max(3, args.steps // 10), 1, dev)
    b14p = bench_block("14b", max(3, args.steps // 10), 1, dev, form="qkpv8")
    xch = bench_exchange(max(5, args.steps // 5), 2, dev)
    stk = bench_stack(max(3, args.steps // 10), 1, dev)
    stk14 = bench_stack(3, 1, dev, "14b")
    dit = bench_dit(max(3, args.steps // 10), 1, dev)
    ditp = bench_dit(max(3, args.steps // 10), 1, dev, form="qkpv8")
    gen = bench_generate(1, 1, dev)
    gdat = bench_gemm_data(max(3, args.steps // 20), 2, dev)
    adat = bench_attention_data(max(5, args.steps // 5), 2, dev, repeats=1)
    libr = bench_library(max(5, args.steps // 5), 2, dev)
    cpu = None if args.no_cpu_baseline else cpu_baseline_kv()
    cpu_extra = None if args.no_cpu_baseline else cpu_baseline_extra()
    # one launch per step: the launch duration is the step time
    achieved = kv["bytes_per_step"] / (kv["ms_pack"] * 1e-3) / 1e9
    line = {
        "metric": "W8A8 GEMM TOPS; FP8 KV pack GB/s; DiT-block ms per 3-frame chunk (1.3B)",
        "value": round(kv["pack_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(kv["ms_pack"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16->e4m3fn",
        "data": "synthetic (seeded CPU generators, Student-t(3) head-dim outliers)",
        "config": {
            "workload": "fp8_kv_pack_30_layers",
            "layers": LAYERS, "tokens": TOKENS, "heads": HEADS, "head_dim": HEAD_DIM,
            "page_tokens": PAGE, "pool_pages": 2 * LAYERS * (TOKENS // PAGE),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic("fp8_kv_pack_30_layers"),
        },
        "cpu_baseline": cpu,
        "cpu_baseline_extra": cpu_extra,
        "extra": {
            "fp8_kv_unpack_gbs": round(kv["unpack_gbs"], 2),
            "fp8_kv_unpack_frac": round(kv["unpack_gbs"] / HBM_PEAK_GBS, 4),
            "fp8_kv_pack_per_layer_launch_gbs": round(kv["pack_layers_gbs"], 2),
            "fp8_kv_unpack_per_layer_launch_gbs": round(kv["unpack_layers_gbs"], 2),
            "kv_pack_us_per_layer_launch": round(kv["ms_pack_layers"] * 1e3 / LAYERS, 3),
            "kv_unpack_us_per_layer_launch": round(kv["ms_unpack_layers"] * 1e3 / LAYERS, 3),
            "w8a8_gemm_tops": round(gm["tops_gemm"], 1),
            "w8a8_gemm_us": round(gm["ms_gemm"] * 1e3, 2),
            "w8a8_gemm_roofline": {"bound": "mfma", "achieved": round(gm["tops_gemm"], 1), "peak": INT8_PEAK_TOPS,
                                   "unit": "TOPS", "frac": round(gm["tops_gemm"] / INT8_PEAK_TOPS, 4)},
            "w8a8_linear_tops_incl_act_quant": round(gm["tops_linear"], 1),
            "w8a8_linear_us_incl_act_quant": round(gm["ms_linear"] * 1e3, 2),
            "w8a8_shape": "x[4680,1536] . W[1536,1536]^T int8, per-token/per-channel scales, bias, bf16 out",
            "fp8_pertensor_gemm_tops": round(gm["tops_fp8_gemm"], 1),
            "fp8_pertensor_gemm_us": round(gm["ms_fp8_gemm"] * 1e3, 2),
            "fp8_pertensor_gemm_roofline": {"bound": "mfma", "achieved": round(gm["tops_fp8_gemm"], 1),
                                            "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                                            "frac": round(gm["tops_fp8_gemm"] / FP8_PEAK_TFLOPS, 4)},
            "fp8_pertensor_linear_us_incl_act_quant": round(gm["ms_fp8_linear"] * 1e3, 2),
            "fp8_pertensor_shape": "the same linear as WaveFp8Linear: e4m3 per-tensor scales (activation scale in "
                                   "bf16 arithmetic), fp32 accumulation, bias, bf16 out",
            "w8a8_block_linears_1p3b_tops": round(lin["tops"], 1),
            "w8a8_block_linears_1p3b_us": round(lin["ms"] * 1e3, 2),
            "w8a8_block_linears_1p3b_frac": round(lin["tops"] / INT8_PEAK_TOPS, 4),
            "w8a8_block_linears_shape": "QKV 4608x1536, O 1536x1536, fc_in 8960x1536, fc_out 1536x8960 on 4680 "
                                        "tokens; 345.97 G int8 ops (the GELU runs in fc_out's input quantizer)",
            "attn_paged_fp8_ms": round(at["ms"], 4),
            "attn_paged_fp8_roofline": {"bound": "mfma", "achieved": round(at["tflops"], 1), "peak": BF16_PEAK_TFLOPS,
                                        "unit": "TFLOP/s", "frac": round(at["tflops"] / BF16_PEAK_TFLOPS, 4)},
            "attn_shape": "Q[4680,12,128] bf16 over 37440 keys (8 chunks) of FP8 e4m3fn pages, bf16 MFMA",
            "attn_paged_fp8_qk8_ms": round(at_qk["ms"], 4),
            "attn_paged_fp8_qk8_tflops": round(at_qk["tflops"], 1),
            "attn_qk8_note": "the quantized-QK backend (hip_fp8_qk, the SageAttention counterpart): per-query e4m3 "
                             "Q against the pages' K codes on the fp8 matrix cores, exact V; same workload",
            "dit_block_1p3b_qk8_ms_per_chunk": round(b13q["ms"], 4),
            "attn_paged_fp8_qkpv8_ms": round(at_pv["ms"], 4),
            "attn_paged_fp8_qkpv8_tflops": round(at_pv["tflops"], 1),
            "attn_qkpv8_note": "the fp8-PV backend (hip_fp8_qkpv, the form of Sage's fp8 P.V kernels): the "
                               "quantized-QK form with e4m3 weights p s_v (a power-of-two scale per query and "
                               "64-key tile) against the pages' V codes on the fp8 matrix cores; same workload",
            "dit_block_1p3b_qkpv8_ms_per_chunk": round(b13p["ms"], 4),
            "fp8_kv_pertensor_layer_us": round(kvt["us_round_trip"], 2),
            "fp8_kv_pertensor_gbs": round(kvt["gbs"], 1),
            "fp8_kv_pertensor_note": "the reference's per-tensor FP8 KV mode (_all_gather_fp8) on one layer's "
                                     "K/V [2,4680,12,128]: amax + quantize (two launches) + fp32 dequant",
            "attn_paged_fp8_context_sweep": {f"{c}_chunks": {"keys": r["keys"], "ms": round(r["ms"], 4),
                                                              "tflops": round(r["tflops"], 1)}
                                             for c, r in at_sweep.items()},
            "exchange_1p3b_ms_per_tick": round(xch["ms_per_tick"], 4),
            "exchange_1p3b_us_per_pass_layer": round(xch["us_per_pass_layer"], 2),
            "exchange_1p3b_gbs": round(xch["gbs"], 1),
            "exchange_note": "paged exchange of one steady-state tick (rf_step 4, 21-frame window): 5 passes x 30 "
                             "layers of K/V packs into the passes' slots + 2 anchor re-RoPE packs over all layers "
                             "(7.85 GB algorithmic); rank 0's context anchor + 2 working + live + self + 3 "
                             "in-flight = 37440 keys",
            "dit_stack_1p3b_ms_per_chunk": round(stk["ms"], 3),
            "dit_stack_1p3b_ms_per_layer": round(stk["ms_per_layer"], 4),
            "dit_stack_1p3b_tokens_per_s": round(stk["tokens_per_s"], 1),
            "dit_stack_1p3b_ms_per_tick_5_passes": round(stk["ms_per_tick_5_passes"], 3),
            "dit_stack_1p3b_ms_per_tick_5_passes_concurrent": round(stk["ms_per_tick_5_passes_concurrent"], 3),
            "dit_stack_14b_ms_per_chunk": round(stk14["ms"], 2),
            "dit_stack_14b_ms_per_layer": round(stk14["ms_per_layer"], 3),
            "dit_stack_14b_ms_per_tick_5_passes": round(stk14["ms_per_tick_5_passes"], 2),
            "dit_stack_14b_ms_per_tick_5_passes_concurrent": round(stk14["ms_per_tick_5_passes_concurrent"], 2),
            "dit_stack_note": "30 blocks of Wan-1.3B (40 of 14B) over one 4680-token chunk: rank 0's denoise pass at a "
                              "steady-state wavefront tick (rf_step 4, 21-frame window; context anchor + 2 working + "
                              "live + self + 3 in-flight = 37440 keys, fused in-block K/V pack per layer), and the "
                              "whole tick (store pass + 4 denoise passes, 2 anchor re-RoPEs); random init drawn on "
                              "the GPU",
            "dit_forward_1p3b_ms_per_chunk": round(dit["ms"], 3),
            "dit_forward_1p3b_tokens_per_s": round(dit["tokens_per_s"], 1),
            "dit_forward_1p3b_qkpv8_ms_per_chunk": round(ditp["ms"], 3),
            "dit_forward_1p3b_qkpv8_tokens_per_s": round(ditp["tokens_per_s"], 1),
            "dit_forward_note": "the whole Wan-1.3B DiT forward of one chunk, noisy latent [1,16,3,60,104] -> x0 "
                                "(patch embedding, time embedding, 30 blocks, head, unpatchify, flow -> x0) as rank "
                                "0's pass of the same steady-state tick (37440-key context), timestep 1000",
            "generate_1p3b_ms_per_stream": round(gen["ms_per_stream"], 1),
            "generate_1p3b_ms_per_tick_mean": round(gen["ms_per_tick_mean"], 2),
            "generate_1p3b_latent_frames_per_s": round(gen["latent_frames_per_s"], 2),
            "generate_note": f"WavefrontDenoiser.generate of a {gen['chunks']}-chunk stream (latent "
                             f"{gen['latent']}) from noise to clean latents: {gen['ticks']} ticks of the store pass "
                             "and the active denoise ranks as a layer wavefront through the 30-block 1.3B DiT, "
                             "re-noising between DMD steps included; ramp-up and drain ticks hold fewer passes",
            "dit_block_1p3b_ms_per_chunk": round(b13["ms"], 4),
            "dit_block_14b_ms_per_chunk": round(b14["ms"], 4),
            "dit_block_14b_qkpv8_ms_per_chunk": round(b14p["ms"], 4),
            "dit_block_note": "one block, 4680-token 3-frame chunk, 37440-key FP8 paged self-attn context, "
                              "512-token text cross-attn, all linears W8A8 int8, random init; includes a 9.4/31 MB "
                              "copy to reset x each step",
            "w8a8_gemm_power": {**gdat, "note": "the int8 GEMM on uniform random int8 operands and with A or W all "
                                                "zero (the same instructions, addresses and bytes), each after a "
                                                "second of sustained launches: the clock under the power limit "
                                                "depends on the operands' switching"},
            "attn_power": {**{k.replace("_ms_0", "_ms"): v for k, v in adat.items()},
                           "note": "the three attention forms on the attention workload with N(0,1) or zero K / V "
                                   "in the pages, each after a second of sustained launches"},
            "library": libr,
        },
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
