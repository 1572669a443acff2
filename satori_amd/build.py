"""Builds satori_amd/libsatori_hip.so (gfx950) from satori_amd/csrc with hipcc.

Every HIP translation unit is compiled with:
  -ffp-contract=off   so no multiply-add is fused unless written as fma (the Q8_K quantizer and the
                      integer products' FP32 epilogue must round exactly like the reference);
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      so the compiler never forms packed FP32 instructions.
Run ``python -m satori_amd.build`` or call ``build()``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libsatori_hip.so")
BUILD_DIR = os.path.join(HERE, "_build")
ARCH = "gfx950"

SOURCES = ["satori_hip.hip", "gemv_float.hip", "gemv_t2.hip", "gemv_kint.hip", "gemv_kmfma.hip", "gemv_fbatch.hip",
           "scale_check.hip", "host_copy.hip", "upload.hip",
           "transformer_ops.hip",
           "host_cpu.cpp", "gguf.cpp"]

COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wno-unused-function"]
HIP_ONLY = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-fno-gpu-rdc"]
# Per-file additions. The matrix-core product consumes its MFMA results on the VALU: the VGPR form of the
# MFMA instructions writes them where the VALU reads them (no accumulator-register copies).
EXTRA = {"gemv_kmfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build libsatori_hip.so")
    return path


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    path = os.path.join(CSRC, src)
    if src.endswith(".hip"):
        cmd = [hipcc(), *HIP_ONLY, *COMMON, *EXTRA.get(src, []), "-c", path, "-o", obj]
    else:
        cmd = [hipcc(), *COMMON, "-c", path, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as pool:
        objects = list(pool.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objects]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
