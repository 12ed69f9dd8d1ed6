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
# Host code built with AddressSanitizer and UndefinedBehaviorSanitizer (device
# code unchanged). Load it with MLXHIP_LIB and the sanitizer runtime preloaded
# (SANITIZER_RUNTIME); tests/test_sanitizers.py does so.
SAN_BUILD = os.path.join(HERE, "_sanitize", "obj")
SAN_LIB = os.path.join(HERE, "_sanitize", "libmlxhip.so")
SANITIZE = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
            "-Xarch_host", "-g"]


def sanitizer_runtime() -> str:
    """The shared ASan runtime of the ROCm clang that compiled the host code
    (it also carries the UBSan handlers)."""
    import glob
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        raise RuntimeError("libclang_rt.asan-x86_64.so not found under /opt/rocm/llvm")
    return hits[-1]

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
    "kernels/gemm_thin.hip",
    "kernels/gemm_bf16.hip",
    "kernels/gemm_f16.hip",
    "kernels/gemm_f32.hip",
    "kernels/gemm16_bf16.hip",
    "kernels/gemm16_f16.hip",
    "kernels/gemm16_x6.hip",
    "kernels/gemm16_small.hip",
    "kernels/decode.hip",
    "kernels/attention.hip",
    "kernels/attention_bwd.hip",
]


# Per-source flags. The attention kernel rescales its MFMA accumulators with
# VALU multiplies every key tile; in the VGPR form of the MFMA instructions
# they are not copied to and from the accumulation registers for that.
EXTRA = {
    "kernels/attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _compile(src: str, sanitize: bool = False) -> tuple[str, float]:
    path = os.path.join(CSRC, src)
    obj = os.path.join(SAN_BUILD if sanitize else BUILD, src.replace("/", "_") + ".o")
    extra = SANITIZE if sanitize else []
    cmd = [HIPCC, f"--offload-arch={ARCH}", *COMMON, *extra, *EXTRA.get(src, []), "-c", path, "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC, "-x", "hip", f"--offload-arch={ARCH}", *COMMON, *extra, "-c", path, "-o", obj]
    t = time.time()
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj, time.time() - t


def build(jobs: int | None = None, verbose: bool = True, sanitize: bool = False) -> str:
    """Compiles every source (always, no staleness check) and links the
    library; with ``sanitize`` the host code is instrumented (ASan + UBSan)
    and the library goes to ``_sanitize/libmlxhip.so``."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(SAN_BUILD if sanitize else BUILD, exist_ok=True)
    jobs = jobs or min(len(SOURCES), max(1, (os.cpu_count() or 4)))
    t0 = time.time()
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = []
        for src, (obj, dt) in zip(SOURCES, ex.map(lambda f: _compile(f, sanitize), SOURCES)):
            objs.append(obj)
            if verbose:
                print(f"  compiled {src}{' (sanitized host code)' if sanitize else ''} in {dt:.1f}s", flush=True)
    lib_path = SAN_LIB if sanitize else LIB
    tmp = lib_path + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, lib_path)
    if verbose:
        print(f"  built {lib_path} in {time.time() - t0:.1f}s", flush=True)
    return lib_path


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)
    if os.path.exists(LIB):
        os.remove(LIB)


if __name__ == "__main__":
    build(sanitize="--sanitize" in sys.argv[1:])
    sys.exit(0)
