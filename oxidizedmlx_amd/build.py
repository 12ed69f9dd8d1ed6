"""Builds libmlxhip.so in-tree with hipcc for gfx950.

Every HIP source is compiled to an object in ``oxidizedmlx_amd/_build`` (in
parallel), then linked into ``oxidizedmlx_amd/libmlxhip.so``. Run as
``python -m oxidizedmlx_amd.build`` or through ``__graft_entry__.build()``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmlxhip.so")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-FP32 instructions are disabled for all device code.
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

SOURCES = [
    "backend.cpp",
    "stream.cpp",
    "autograd.cpp",
    "decoder.cpp",
    "kernels/rows.hip",
    "kernels/elementwise.hip",
    "kernels/gemm.hip",
    "kernels/gemm_small.hip",
    "kernels/gemm_bf16.hip",
    "kernels/gemm_f16.hip",
    "kernels/gemm_f32.hip",
    "kernels/gemm16_bf16.hip",
    "kernels/gemm16_f16.hip",
    "kernels/decode.hip",
    "kernels/attention.hip",
]


# Per-source flags. The attention kernel rescales its MFMA accumulators with
# VALU multiplies every key tile; in the VGPR form of the MFMA instructions
# they are not copied to and from the accumulation registers for that.
EXTRA = {
    "kernels/attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _compile(src: str) -> tuple[str, float]:
    path = os.path.join(CSRC, src)
    obj = os.path.join(BUILD, src.replace("/", "_") + ".o")
    cmd = [HIPCC, f"--offload-arch={ARCH}", *COMMON, *EXTRA.get(src, []), "-c", path, "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC, "-x", "hip", f"--offload-arch={ARCH}", *COMMON, "-c", path, "-o", obj]
    t = time.time()
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj, time.time() - t


def build(jobs: int | None = None, verbose: bool = True) -> str:
    """Compiles every source (always, no staleness check) and links the library."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(SOURCES), max(1, (os.cpu_count() or 4)))
    t0 = time.time()
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = []
        for src, (obj, dt) in zip(SOURCES, ex.map(_compile, SOURCES)):
            objs.append(obj)
            if verbose:
                print(f"  compiled {src} in {dt:.1f}s", flush=True)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"  built {LIB} in {time.time() - t0:.1f}s", flush=True)
    return LIB


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)
    if os.path.exists(LIB):
        os.remove(LIB)


if __name__ == "__main__":
    build()
    sys.exit(0)
