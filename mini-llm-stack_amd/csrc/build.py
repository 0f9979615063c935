"""Builds libmls_hip.so (gfx950 code objects + C ABI) next to the package.

    python mini-llm-stack_amd/csrc/build.py [--jobs N] [--verbose]

Each .hip file is compiled by hipcc for --offload-arch=gfx950 into an object
file under csrc/_build/, then linked into ../libmls_hip.so. Packed-fp32 VALU
instructions are disabled for all device code (-packed-fp32-ops). bench.py's
calibration kernels (floor.hip) go into a separate ../libmls_floor.so.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
OUT = PKG / "libmls_hip.so"
BUILD = CSRC / "_build"
SOURCES = ["abi.hip", "e4m3.hip", "quant.hip", "gemv.hip", "gemv_mfma.hip", "gemv_mfma8.hip", "gemm_mfma16.hip", "gemm_grouped.hip",
           "wq_abi.hip", "gemm_small.hip", "gemm_bytes.hip", "gemm_fp8.hip", "dgrad.hip", "moe.hip", "transpose.hip", "paged_attn.hip", "split.hip"]
ARCH = "gfx950"
# Per-source device-code options.
# - Kernel-argument preloading (gemv.hip, gemv_mfma*.hip, gemm_small.hip, split.hip, and
#   bench.py's calibration kernels in floor.hip): the first 14 dwords of a kernel's arguments arrive in SGPRs at wavefront
#   start, so the microsecond kernels issue their first loads without a scalar-load round
#   trip for the arguments (their argument lists put what those loads need first). The code
#   object keeps a prologue that loads them for firmware without preloading.
# - gemv_mfma.hip (the skinny GEMM's INT4 kernels), gemm_small.hip, gemm_grouped.hip: MFMA
#   results in VGPRs (the kernels scale MFMA results with VALU FMAs; in AGPRs each one is
#   first copied back with v_accvgpr_read, 56 extra VALU instructions per wavefront in the
#   skinny kernel at K = 4096). The skinny INT8 kernels (gemv_mfma8.hip) measured slower
#   that way and keep the default.
PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=16"]
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
EXTRA_FLAGS = {"gemv.hip": PRELOAD,
               "floor.hip": PRELOAD,
               "gemv_mfma.hip": VGPR_FORM + PRELOAD,
               "gemv_mfma8.hip": PRELOAD,
               "gemm_small.hip": VGPR_FORM + PRELOAD,
               "gemm_grouped.hip": VGPR_FORM,
               "split.hip": PRELOAD}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def common_flags() -> list[str]:
    return ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
            "-Wno-unused-command-line-argument",
            f"-I{CSRC}", f"-I{PKG.parent / 'include'}"]


def compile_one(src: str, verbose: bool) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    cmd = [hipcc(), *common_flags(), *EXTRA_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, flush=True)
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: compile_one(s, verbose), SOURCES))
    tmp = OUT.with_suffix(".so.tmp")
    # --no-undefined: a kernel whose host-side launch stub was not emitted must fail
    # the build here, not the first dlopen
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-Wl,--no-undefined", "-o", str(tmp),
           *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, OUT)
    build_floor(verbose)
    return OUT


FLOOR_OUT = PKG / "libmls_floor.so"


def build_floor(verbose: bool = False) -> Path:
    """libmls_floor.so: bench.py's single-launch calibration kernels (floor.hip), kept
    out of the library and its ABI."""
    obj = compile_one("floor.hip", verbose)
    tmp = FLOOR_OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-Wl,--no-undefined", "-o", str(tmp), str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed (floor):\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, FLOOR_OUT)
    return FLOOR_OUT


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    out = build(args.jobs, args.verbose)
    print(f"built {out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
