"""Benchmark of the quantized DiT-block path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Headline workload: FP8 e4m3fn KV pack of 30 layers of the Wan-1.3B chunk
(K and V bf16 [4680, 12, 128] per layer, heavy-tailed, per-(token, head)
scales, 1560-token pages at seeded random page-table slots).  One step packs
all 30 layers (one kernel launch per layer, as the exchange publishes one
layer at a time); inputs are resident in HBM before the timed region.
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
LAYERS, TOKENS, HEADS, HEAD_DIM, PAGE = 30, 4680, 12, 128, 1560


def kv_bytes_per_layer() -> int:
    """Algorithmic bytes of packing (or unpacking) one layer's K and V."""
    elems = TOKENS * HEADS * HEAD_DIM
    rows = TOKENS * HEADS
    return 2 * (elems * 2 + elems * 1 + rows * 4)


def _timed(fn, steps: int, warmup: int) -> float:
    """Mean ms per call of ``fn`` over ``steps`` calls, bracketed by HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def bench_kv(steps: int, warmup: int, dev: str):
    ppl = TOKENS // PAGE
    pool_pages = 2 * LAYERS * ppl
    ids = inputs.page_table(LAYERS * ppl, pool_pages, seed=7)
    pool = Fp8PagePool(pool_pages, HEADS, HEAD_DIM, PAGE, dev)
    tables = [pool.page_table(ids[i * ppl:(i + 1) * ppl]) for i in range(LAYERS)]
    ks, vs = [], []
    for layer in range(LAYERS):
        k, v = inputs.kv_layer(layer)
        ks.append(k.to(dev))
        vs.append(v.to(dev))
    outk = torch.empty((TOKENS, HEADS, HEAD_DIM), dtype=torch.bfloat16, device=dev)
    outv = torch.empty_like(outk)

    def pack_step():
        for layer in range(LAYERS):
            pool.pack(ks[layer], vs[layer], tables[layer])

    def unpack_step():
        for layer in range(LAYERS):
            pool.unpack(tables[layer], TOKENS, out_k=outk, out_v=outv)

    ms_pack = _timed(pack_step, steps, warmup)
    ms_unpack = _timed(unpack_step, steps, warmup)
    step_bytes = LAYERS * kv_bytes_per_layer()
    return {
        "ms_pack": ms_pack,
        "ms_unpack": ms_unpack,
        "pack_gbs": step_bytes / (ms_pack * 1e-3) / 1e9,
        "unpack_gbs": step_bytes / (ms_unpack * 1e-3) / 1e9,
        "launch_us_pack": ms_pack * 1e3 / LAYERS,
        "launch_us_unpack": ms_unpack * 1e3 / LAYERS,
        "bytes_per_launch": kv_bytes_per_layer(),
    }


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
        "cores": threads,
        "kind": "port",
        "sample": f"oracle torch-CPU pack of {n_layers} of the 30 layers (K and V), median of {len(reps)} reps",
    }


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the path runs on a single GPU); --gpus {args.gpus} is not supported",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = "cuda:0"
    kv = bench_kv(args.steps, args.warmup, dev)
    cpu = None if args.no_cpu_baseline else cpu_baseline_kv()
    achieved = kv["bytes_per_launch"] / (kv["launch_us_pack"] * 1e-6) / 1e9
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
            "traffic": None,
        },
        "cpu_baseline": cpu,
        "extra": {
            "fp8_kv_unpack_gbs": round(kv["unpack_gbs"], 2),
            "fp8_kv_unpack_frac": round(kv["unpack_gbs"] / HBM_PEAK_GBS, 4),
            "kv_pack_us_per_layer": round(kv["launch_us_pack"], 3),
            "kv_unpack_us_per_layer": round(kv["launch_us_unpack"], 3),
        },
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
