"""Builds libgmmxx_hip.so for gfx950 in-tree with hipcc.

    python -m gmmxx_amd.build          # or: from gmmxx_amd.build import build; build()

Each translation unit is compiled separately (in parallel) and linked into a
shared library next to this file, where ``gmmxx_amd._hip`` loads it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libgmmxx_hip.so")
SOURCES = ("em_tile.hip", "em_sph_bf16.hip", "em_fused.hip", "em_coop.hip", "em_full_wide.hip", "em_full_infer.hip",
           "params.hip",
           "kmeans.hip", "abi.hip")
ARCH = os.environ.get("GMMXX_HIP_ARCH", "gfx950")

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", CSRC, "-I", os.path.join(ROOT, "include"),
]
# The tile kernels' logits are finite or -inf: no NaN canonicalisation around
# min/max there.  Kept off elsewhere (the Cholesky kernel tests for NaN pivots).
EXTRA_FLAGS = {"em_tile.hip": ["-fno-honor-nans", "-mno-amdgpu-ieee"],
               "em_sph_bf16.hip": ["-fno-honor-nans", "-mno-amdgpu-ieee"],
               "em_fused.hip": ["-fno-honor-nans", "-mno-amdgpu-ieee"],
               "em_coop.hip": ["-fno-honor-nans", "-mno-amdgpu-ieee"]}


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return path


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *COMMON_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every HIP translation unit and link libgmmxx_hip.so; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
