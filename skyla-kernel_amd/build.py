"""Builds libskyla_hip.so: the gfx950 code objects, embedded into the C-ABI runtime.

    python skyla-kernel_amd/build.py

Steps (all in-tree, no JIT cache):
  1. hipcc --genco --offload-arch=gfx950 for every csrc/kernels/*.hip -> build/*.hsaco
  2. the code objects are assembled into build/embed.o (csrc/runtime/embed.S, .incbin)
  3. the host runtime csrc/runtime/skyla_hip.cpp + embed.o -> lib/libskyla_hip.so
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "build")
LIB_DIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIB_DIR, "libskyla_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
KERNELS = ("matvec", "matmul", "moe", "util", "attention")

# Packed FP32 instructions are disabled for all device code; f16 packed math is kept.
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "--genco",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def hipcc() -> str:
    path = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; set ROCM_PATH")
    return path


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    cc = hipcc()
    jobs = []
    for k in KERNELS:
        src = os.path.join(CSRC, "kernels", f"{k}.hip")
        out = os.path.join(BUILD, f"{k}.hsaco")
        jobs.append([cc, *HIP_FLAGS, "-o", out, src])
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        for f in [ex.submit(_run, j) for j in jobs]:
            f.result()
    embed_o = os.path.join(BUILD, "embed.o")
    _run(["gcc", "-c", "-I", BUILD, "-o", embed_o, os.path.join(CSRC, "runtime", "embed.S")])
    tmp = LIB + ".tmp"
    _run([
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
        "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"),
        "-o", tmp, os.path.join(CSRC, "runtime", "skyla_hip.cpp"), embed_o,
        "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}",
        "-Wl,--no-undefined",
    ])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
