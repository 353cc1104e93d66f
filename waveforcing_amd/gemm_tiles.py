"""A/B of the W8A8 GEMM's two workgroup tiles from the instrumented build.

Usage: python -m waveforcing_amd.build --variant gemm_tiles        (on the CPU, once)
       python -m waveforcing_amd.gemm_tiles [--fp8] [--block]      (on the GPU)

The instrumented library (libwf_mi355x_gemm_tiles.so, built with -DWF_GEMM_TILE_LAB) has the product's
kernels plus wf_gemm_set_tile_policy, which forces the tile plan of the following launches: 0 the 128 x 256
tile (three 48 KB LDS stages) over the whole output, 1 the 256 x 256 tile (two 64 KB stages) over the whole
output, -1 the product's plan (one of those, or whole rounds of 256 x 256 tiles followed by a launch of
128 x 256 tiles over the rest).  For each Wan-1.3B / 14B linear at 4680 tokens (uniform random int8
operands, or random e4m3 codes with --fp8) it checks that the three give bit-identical outputs (every
output's accumulator sees the same MFMAs in the same K order; int8 also compares the int32 accumulators)
and times them in alternating blocks after a second of warm-up, so that all run in the same power and clock
state.  With --block it runs, instead, the 1.3B block's four linears, the 1.3B block and the 14B block
(bench.py's workloads) under the product's plan against the 128-row tile everywhere, alternating.  One JSON
line per result.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import statistics
import time

import torch

from .build import variant_path

M = 4680
SHAPES = [("1.3B QKV", 4608, 1536), ("1.3B O", 1536, 1536), ("1.3B fc_in", 8960, 1536), ("1.3B fc_out", 1536, 8960),
          ("14B QKV", 15360, 5120), ("14B O", 5120, 5120), ("14B fc_in", 13824, 5120), ("14B fc_out", 5120, 13824)]


def _lab():
    lib = ctypes.CDLL(variant_path("gemm_tiles"))
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    lib.wf_gemm_i8.argtypes = [vp, vp, i64, i64, i64, vp, vp, vp, vp, i64, vp, i32, vp]
    lib.wf_gemm_fp8_pertensor.argtypes = [vp, vp, i64, i64, i64, vp, vp, vp, vp, i64, vp]
    lib.wf_gemm_set_tile_policy.argtypes = [i32]
    return lib


def shapes_ab(fp8: bool, dev: str = "cuda:0") -> None:
    lib = _lab()

    def call(policy, a, w, sx, sw, bias, y, acc):
        assert lib.wf_gemm_set_tile_policy(policy) == 0
        N, K = w.shape
        if fp8:
            rc = lib.wf_gemm_fp8_pertensor(a.data_ptr(), w.data_ptr(), M, N, K, sx.data_ptr(), sw.data_ptr(),
                                           bias.data_ptr(), y.data_ptr(), y.stride(0), None)
        else:
            rc = lib.wf_gemm_i8(a.data_ptr(), w.data_ptr(), M, N, K, sx.data_ptr(), sw.data_ptr(), bias.data_ptr(),
                                y.data_ptr(), y.stride(0), None if acc is None else acc.data_ptr(), 0, None)
        if rc != 0:
            raise RuntimeError(f"GEMM launch failed with status {rc}")

    for name, N, K in SHAPES:
        print(f"[case] {name} {M}x{N}x{K} fp8={fp8}", flush=True)
        g = torch.Generator(device=dev).manual_seed(N + K)
        if fp8:
            # uniformly random e4m3 codes, NaN codes (0x7f, 0xff) replaced by 0x7e / 0xfe
            a = torch.randint(0, 256, (M, K), generator=g, device=dev, dtype=torch.int32)
            w = torch.randint(0, 256, (N, K), generator=g, device=dev, dtype=torch.int32)
            a = torch.where((a & 0x7f) == 0x7f, a - 1, a).to(torch.uint8)
            w = torch.where((w & 0x7f) == 0x7f, w - 1, w).to(torch.uint8)
            sx = torch.full((1,), 0.01, device=dev)
            sw = torch.full((1,), 0.02, device=dev)
        else:
            a = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int32).to(torch.int8)
            w = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int32).to(torch.int8)
            sx = torch.rand((M,), generator=g, device=dev) * 0.01
            sw = torch.rand((N,), generator=g, device=dev) * 0.01
        bias = torch.randn((N,), generator=g, device=dev).to(torch.bfloat16)
        pols = (0, 1, -1)
        ys = {pol: torch.full((M, N), 7.0, dtype=torch.bfloat16, device=dev) for pol in pols}
        accs = {pol: None if fp8 else torch.full((M, N), 7, dtype=torch.int32, device=dev) for pol in pols}
        for pol in pols:
            call(pol, a, w, sx, sw, bias, ys[pol], accs[pol])
        torch.cuda.synchronize()
        same = all(bool(torch.equal(ys[0], ys[pol])) and (fp8 or bool(torch.equal(accs[0], accs[pol])))
                   for pol in pols[1:])
        ops = 2.0 * M * N * K
        reps = max(3, int(4e11 / ops))
        t0 = time.time()
        while time.time() - t0 < 1.0:
            for pol in pols:
                call(pol, a, w, sx, sw, bias, ys[pol], None)
            torch.cuda.synchronize()
        times = {pol: [] for pol in pols}
        for blk in range(6):
            for pol in (pols if blk % 2 == 0 else pols[::-1]):
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                for _ in range(reps):
                    call(pol, a, w, sx, sw, bias, ys[pol], None)
                e.record()
                torch.cuda.synchronize()
                times[pol].append(s.elapsed_time(e) / reps * 1e3)
        med = {p: statistics.median(t) for p, t in times.items()}
        print(json.dumps({"shape": name, "M": M, "N": N, "K": K, "fp8": fp8, "bit_identical": same,
                          "tiles_128": -(-M // 128) * -(-N // 256), "tiles_256": -(-M // 256) * -(-N // 256),
                          "us_128": round(med[0], 2), "us_256": round(med[1], 2), "us_plan": round(med[-1], 2),
                          "tops_128": round(ops / med[0] / 1e6, 1), "tops_256": round(ops / med[1] / 1e6, 1),
                          "tops_plan": round(ops / med[-1] / 1e6, 1),
                          "ratio_256_over_128": round(med[1] / med[0], 4),
                          "ratio_plan_over_128": round(med[-1] / med[0], 4)}), flush=True)
        if not same:
            raise RuntimeError(f"{name}: the tile plans disagree")
        del a, w, ys, accs


def block_ab(dev: str = "cuda:0") -> None:
    import os
    import sys

    from . import _lib

    torch.zeros(1, device=dev)
    _lib.LIB_PATH = variant_path("gemm_tiles")
    lib = _lib.load()
    lib.wf_gemm_set_tile_policy.argtypes = [ctypes.c_int32]
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench

    for rep in range(3):
        for pol in ((0, -1) if rep % 2 == 0 else (-1, 0)):
            assert lib.wf_gemm_set_tile_policy(pol) == 0
            lin = bench.bench_block_linears(20, 3, dev)
            blk = bench.bench_block("1.3b", 20, 3, dev)
            b14 = bench.bench_block("14b", 10, 2, dev)
            print(json.dumps({"rep": rep, "policy": "product plan" if pol < 0 else "128-row tile",
                              "linears_1p3b_us": round(lin["ms"] * 1e3, 1), "linears_1p3b_tops": round(lin["tops"], 1),
                              "block_1p3b_ms": round(blk["ms"], 4), "block_14b_ms": round(b14["ms"], 4)}),
                  flush=True)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--fp8", action="store_true", help="the per-tensor e4m3 GEMM instead of the int8 one")
    ap.add_argument("--block", action="store_true", help="the 1.3B block's linears and the block instead")
    args = ap.parse_args()
    if args.block:
        block_ab()
    else:
        shapes_ab(args.fp8)


if __name__ == "__main__":
    main()
