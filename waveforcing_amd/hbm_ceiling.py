"""The HBM ceiling for the FP8 KV pack's traffic mix, from the instrumented build.

Usage: python -m waveforcing_amd.build --variant hbm_probe      (on the CPU, once)
       python -m waveforcing_amd.hbm_ceiling [--reps R]          (on the GPU)

The instrumented library (libwf_mi355x_hbm_probe.so, built with -DWF_HBM_PROBE) holds the product's kernels
plus wf_probe_stream_2to1: a bare grid-stride stream that reads 16 bytes and writes 8 per thread and
iteration, fully coalesced, with plain or nontemporal stores: the pack's 2 : 1 read : write ratio with no
other work.  Over the pack workload's 862.6 MB of input (30 layers of K and V, [4680, 12, 128] bf16) it
sweeps the grid size, then times the 30-layer pack itself in the same process, each after a second of
sustained launches, R times in alternation.  One JSON line per measurement; GB/s count bytes read plus
written.
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
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench

    in_bytes = bench.LAYERS * 2 * bench.TOKENS * bench.HEADS * bench.HEAD_DIM * 2
    n = in_bytes // 16
    src = torch.full((in_bytes // 2,), 0x3C3C, dtype=torch.int16, device=dev)
    dst = torch.empty((in_bytes // 2,), dtype=torch.uint8, device=dev)
    stream = _lib.stream_handle(dev)

    def stream_call(grid, nt):
        rc = lib.wf_probe_stream_2to1(src.data_ptr(), dst.data_ptr(), n, grid, nt, stream)
        if rc != 0:
            raise RuntimeError(f"wf_probe_stream_2to1 failed with status {rc}")

    for rep in range(args.reps):
        best = 0.0
        for nt in (0, 1):
            for grid in GRIDS:
                ms = bench._timed(lambda: stream_call(grid, nt), 20, 3, 1.0)
                gbs = 24.0 * n / (ms * 1e-3) / 1e9
                best = max(best, gbs)
                print(json.dumps({"rep": rep, "kernel": "stream_2to1", "nontemporal": nt, "grid": grid,
                                  "us": round(ms * 1e3, 1), "gbs": round(gbs, 1)}), flush=True)
        kv = bench.bench_kv(20, 3, dev, ("pack",))
        print(json.dumps({"rep": rep, "kernel": "kv_pack 30 layers", "us": round(kv["ms_pack"] * 1e3, 1),
                          "gbs": round(kv["pack_gbs"], 1), "stream_2to1_best_gbs": round(best, 1),
                          "pack_over_stream": round(kv["pack_gbs"] / best, 4)}), flush=True)


if __name__ == "__main__":
    main()
