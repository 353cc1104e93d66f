"""The HBM ceilings for the FP8 KV pack's and unpack's traffic mixes, from the instrumented build.

Usage: python -m waveforcing_amd.build --variant hbm_probe      (on the CPU, once)
       python -m waveforcing_amd.hbm_ceiling [--reps R]          (on the GPU)

The instrumented library (libwf_mi355x_hbm_probe.so, built with -DWF_HBM_PROBE) holds the product's kernels
plus wf_probe_stream_2to1 / wf_probe_stream_1to2: bare grid-stride streams that read 16 bytes and write 8
(or read 8 and write 16) per thread and iteration, fully coalesced, with plain or nontemporal stores: the
pack's 2 : 1 and the unpack's 1 : 2 read : write ratios with no other work.  Over the pack workload's
862.6 MB of bf16 (30 layers of K and V, [4680, 12, 128]) and its 431.3 MB of codes it sweeps the grid size,
then times the 30-layer pack and unpack themselves in the same process, each after a second of sustained
launches, R times in alternation.  One JSON line per measurement; GB/s count bytes read plus written.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys

import torch

from .build import variant_path

GRIDS = (2048, 4096, 8192, 16384, 65536, 131072)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--reps", type=int, default=2)
    args = ap.parse_args()
    dev = "cuda:0"
    torch.zeros(1, device=dev)
    from . import _lib

    _lib.LIB_PATH = variant_path("hbm_probe")
    lib = _lib.load()
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    lib.wf_probe_stream_2to1.argtypes = [vp, vp, i64, i32, i32, vp]
    lib.wf_probe_stream_1to2.argtypes = [vp, vp, i64, i32, i32, vp]
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench

    in_bytes = bench.LAYERS * 2 * bench.TOKENS * bench.HEADS * bench.HEAD_DIM * 2
    n = in_bytes // 16
    src = torch.full((in_bytes // 2,), 0x3C3C, dtype=torch.int16, device=dev)
    dst = torch.empty((in_bytes // 2,), dtype=torch.uint8, device=dev)
    stream = _lib.stream_handle(dev)

    def stream_call(fn, a, b, grid, nt):
        rc = fn(a.data_ptr(), b.data_ptr(), n, grid, nt, stream)
        if rc != 0:
            raise RuntimeError(f"stream probe failed with status {rc}")

    for rep in range(args.reps):
        best = {}
        for name, fn, a, b in (("stream_2to1", lib.wf_probe_stream_2to1, src, dst),
                               ("stream_1to2", lib.wf_probe_stream_1to2, dst, src)):
            best[name] = 0.0
            for nt in (0, 1):
                for grid in GRIDS:
                    ms = bench._timed(lambda: stream_call(fn, a, b, grid, nt), 20, 3, 1.0)
                    gbs = 24.0 * n / (ms * 1e-3) / 1e9
                    best[name] = max(best[name], gbs)
                    print(json.dumps({"rep": rep, "kernel": name, "nontemporal": nt, "grid": grid,
                                      "us": round(ms * 1e3, 1), "gbs": round(gbs, 1)}), flush=True)
        kv = bench.bench_kv(20, 3, dev, ("pack", "unpack"))
        for op, key in (("pack", "stream_2to1"), ("unpack", "stream_1to2")):
            print(json.dumps({"rep": rep, "kernel": f"kv_{op} 30 layers", "us": round(kv[f"ms_{op}"] * 1e3, 1),
                              "gbs": round(kv[f"{op}_gbs"], 1), f"{key}_best_gbs": round(best[key], 1),
                              "over_stream": round(kv[f"{op}_gbs"] / best[key], 4)}), flush=True)


if __name__ == "__main__":
    main()
