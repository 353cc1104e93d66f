"""Phase timing of the W8A8 int8 GEMM from its instrumented build.

Usage: python -m waveforcing_amd.build --variant gemm_phases   (on the CPU, once)
       python -m waveforcing_amd.gemm_phases [--reps R]        (on the GPU)

The instrumented library (libwf_mi355x_gemm_phases.so, built with
-DWF_GEMM_PHASES) has the same kernels as the product library plus shader-clock
stamps that the two waves of SIMD 0 of every workgroup write at kernel entry,
after the prologue barrier, after the K loop's last barrier and after the
epilogue's last store: the shader clock (s_memtime, wave 0) and the 100 MHz
reference clock (s_memrealtime, wave 4).  For each Wan shape this prints, averaged over
the workgroups of R launches (wave 0's stamps): the prologue, the cycles per K step (the K loop
divided by its steps, against the 1024 cycles one step needs on the matrix
cores: 16 v_mfma_i32_32x32x32_i8 of 32 cycles for each of the SIMD's two
waves) and the epilogue, with the launch's event time and the shader clock (a workgroup's
cycles over its reference-clock time, averaged).
With --zero-a the activations are all zero: the same instructions, addresses and bytes, fewer
toggling bits, so the cycle counts stay and only the clock under the power limit moves.  With --fp8 the
per-tensor e4m3 GEMM (wf_gemm_fp8_pertensor: the same kernel with v_mfma_f32_32x32x64_f8f6f4, 8 MFMAs of
64 cycles per wave and K step) runs on uniformly random e4m3 codes instead.  Stamps are compared
only within a workgroup: the shader-clock counters of different XCDs are not
one time base.
"""

from __future__ import annotations

import argparse
import ctypes
import math
import time

import torch

from .build import variant_path

BM, BN, BK, XCD = 128, 256, 128, 8
SHAPES = [  # (name, M, N, K): the Wan-1.3B block's linears and the 14B ones, 4680 tokens
    ("1.3B O / cfg1", 4680, 1536, 1536), ("1.3B QKV", 4680, 4608, 1536), ("1.3B fc_in", 4680, 8960, 1536),
    ("1.3B fc_out", 4680, 1536, 8960), ("14B O", 4680, 5120, 5120), ("14B fc_out", 4680, 5120, 13824),
]


def _lib(path: str | None = None):
    lib = ctypes.CDLL(path or variant_path("gemm_phases"))
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    lib.wf_gemm_i8.argtypes = [vp, vp, i64, i64, i64, vp, vp, vp, vp, i64, vp, i32, vp]
    lib.wf_gemm_fp8_pertensor.argtypes = [vp, vp, i64, i64, i64, vp, vp, vp, vp, i64, vp]
    lib.wf_gemm_set_phase_buffer.argtypes = [vp]
    lib.wf_gemm_set_tile_policy.argtypes = [i32]
    # the stamps below are read as 128 x 256 tiles of 8 waves: force that tile (the product picks the
    # 256 x 256 tile for some shapes; waveforcing_amd.gemm_tiles compares the two)
    if lib.wf_gemm_set_tile_policy(0) != 0:
        raise RuntimeError("wf_gemm_set_tile_policy failed")
    return lib


def measure(lib, M: int, N: int, K: int, reps: int, dev="cuda:0", zero_a: bool = False, fp8: bool = False) -> dict:
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    if fp8:
        # uniformly random e4m3 codes, NaN codes (0x7f, 0xff) replaced by 0x7e / 0xfe
        qx = torch.randint(0, 256, (M, K), generator=g, device=dev, dtype=torch.int32)
        qw = torch.randint(0, 256, (N, K), generator=g, device=dev, dtype=torch.int32)
        qx = torch.where((qx & 0x7f) == 0x7f, qx - 1, qx).to(torch.uint8)
        qw = torch.where((qw & 0x7f) == 0x7f, qw - 1, qw).to(torch.uint8)
    else:
        qx = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
        qw = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
    if zero_a:
        qx.zero_()
    sx = torch.rand((M,), generator=g, device=dev) * 1e-3
    sw = torch.rand((N,), generator=g, device=dev) * 1e-3
    bias = torch.zeros((N,), dtype=torch.bfloat16, device=dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    tiles = math.ceil(M / BM) * math.ceil(N / BN)
    grid = math.ceil(tiles / XCD) * XCD
    stamps = torch.zeros((grid, 8), dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def launch():
        if fp8:
            rc = lib.wf_gemm_fp8_pertensor(qx.data_ptr(), qw.data_ptr(), M, N, K, sx.data_ptr(), sw.data_ptr(),
                                           bias.data_ptr(), y.data_ptr(), N, stream)
        else:
            rc = lib.wf_gemm_i8(qx.data_ptr(), qw.data_ptr(), M, N, K, sx.data_ptr(), sw.data_ptr(), bias.data_ptr(),
                                y.data_ptr(), N, None, 0, stream)
        if rc != 0:
            raise RuntimeError(f"GEMM launch failed with status {rc}")

    lib.wf_gemm_set_phase_buffer(None)
    t0 = time.perf_counter()
    n = 0
    while n < 5 or time.perf_counter() - t0 < 0.5:  # half a second of sustained launches: the clock settles
        launch()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    lib.wf_gemm_set_phase_buffer(stamps.data_ptr())
    rows, times = [], []
    for _ in range(reps):
        stamps.zero_()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        launch()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) * 1e-3)
        rows.append(stamps.cpu())
    lib.wf_gemm_set_phase_buffer(None)
    nk = math.ceil(K / BK)
    pro, step, epi, life = [], [], [], []
    for st in rows:
        live = st[(st > 0).all(dim=1)].double()
        w0 = live[:, 0:4]
        pro.append((w0[:, 1] - w0[:, 0]).mean().item())
        step.append(((w0[:, 2] - w0[:, 1]) / nk).mean().item())
        epi.append((w0[:, 3] - w0[:, 2]).mean().item())
        ref = live[:, 4:8]
        life.append(((w0[:, 3] - w0[:, 0]) / ((ref[:, 3] - ref[:, 0]) * 1e-8)).mean().item())
    mean = lambda v: sum(v) / len(v)  # noqa: E731
    return {"tiles": tiles, "k_steps": nk, "prologue_cycles": mean(pro), "cycles_per_k_step": mean(step),
            "epilogue_cycles": mean(epi), "event_us": mean(times) * 1e6, "mfma_cycles_per_k_step": 1024,
            "clock_ghz": mean(life) / 1e9}


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--lib", default=None, help="another library built with -DWF_GEMM_PHASES (default: the "
                                                "gemm_phases variant of this package)")
    ap.add_argument("--shapes", default=None, help="comma-separated indices into the shape list")
    ap.add_argument("--zero-a", action="store_true", help="all-zero activations (same work, fewer toggling bits)")
    ap.add_argument("--fp8", action="store_true", help="the per-tensor e4m3 GEMM on random e4m3 codes")
    args = ap.parse_args()
    lib = _lib(args.lib)
    shapes = SHAPES if args.shapes is None else [SHAPES[int(i)] for i in args.shapes.split(",")]
    print("| shape | M x N x K | tiles | K steps | prologue (cycles) | cycles / K step (MFMA: 1024) | "
          "epilogue (cycles) | event µs | clock (GHz) |")
    print("|---|---|---:|---:|---:|---:|---:|---:|---:|")
    for name, M, N, K in shapes:
        r = measure(lib, M, N, K, args.reps, zero_a=args.zero_a, fp8=args.fp8)
        print(f"| {name} | {M} x {N} x {K} | {r['tiles']} | {r['k_steps']} | {r['prologue_cycles']:.0f} | "
              f"{r['cycles_per_k_step']:.0f} | {r['epilogue_cycles']:.0f} | {r['event_us']:.2f} | "
              f"{r['clock_ghz']:.2f} |", flush=True)


if __name__ == "__main__":
    main()
