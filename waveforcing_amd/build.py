"""Build libwf_mi355x.so from csrc/*.hip with hipcc for gfx950.

Usage: python -m waveforcing_amd.build [--jobs N] [--verbose] [--variant gemm_phases|gemm_tiles|hbm_probe]

Every translation unit is compiled to an object under waveforcing_amd/_build/
in parallel, then linked into waveforcing_amd/libwf_mi355x.so (in-tree, so it
travels with the source tree).  There is no incremental logic on purpose: a
call always rebuilds.

``--variant gemm_phases`` builds a separate, instrumented library,
libwf_mi355x_gemm_phases.so, whose W8A8 GEMM records shader-clock stamps of its
phases (waveforcing_amd/gemm_phases.py reads them); ``--variant gemm_tiles``
builds libwf_mi355x_gemm_tiles.so, whose GEMM tile can be forced per launch
(wf_gemm_set_tile_policy, for A/B runs of the two workgroup tiles);
``--variant hbm_probe`` builds libwf_mi355x_hbm_probe.so with bare 2 : 1 and
1 : 2 read : write stream kernels (wf_probe_stream_2to1 / _1to2, read by
waveforcing_amd/hbm_ceiling.py).  The product library is built with none.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libwf_mi355x.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = "gfx950"
# instrumented variants: name -> extra compile flags (their own object directory and library name)
VARIANTS = {"gemm_phases": ["-DWF_GEMM_PHASES"], "gemm_tiles": ["-DWF_GEMM_TILE_LAB"], "hbm_probe": ["-DWF_HBM_PROBE"]}

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fno-gpu-rdc",
    "-Wall",
    "-Wno-unused-function",
    # No implicit multiply-add contraction: elementwise fp32 follows the
    # reference's operation order exactly; kernels write fmaf() where they
    # want a fused multiply-add.
    "-ffp-contract=off",
    # Packed FP32 VALU forms are kept out of the generated code.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm is required to build the extension)")
    return path


def _compile(src: str, verbose: bool, build_dir: str = BUILD_DIR, extra: tuple = ()) -> str:
    obj = os.path.join(build_dir, os.path.basename(src) + ".o")
    cmd = [_hipcc(), *COMMON_FLAGS, *extra, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(ln for ln in res.stderr.splitlines() if noise not in ln)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    return obj


def variant_path(variant: str) -> str:
    return os.path.join(PKG_DIR, f"libwf_mi355x_{variant}.so")


def build(jobs: int | None = None, verbose: bool = False, variant: str | None = None) -> str:
    """Compile every csrc/*.hip and link the shared library (or an instrumented ``variant``); return its path."""
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    if variant is not None and variant not in VARIANTS:
        raise ValueError(f"unknown build variant {variant!r} (known: {sorted(VARIANTS)})")
    build_dir = BUILD_DIR if variant is None else os.path.join(BUILD_DIR, variant)
    lib_path = LIB_PATH if variant is None else variant_path(variant)
    extra = () if variant is None else tuple(VARIANTS[variant])
    os.makedirs(build_dir, exist_ok=True)
    jobs = jobs or min(8, len(srcs), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose, build_dir, extra), srcs))
    tmp = lib_path + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-fno-gpu-rdc", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, lib_path)
    return lib_path


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--variant", choices=sorted(VARIANTS), default=None)
    args = ap.parse_args()
    print(build(args.jobs, args.verbose, args.variant))


if __name__ == "__main__":
    main()
