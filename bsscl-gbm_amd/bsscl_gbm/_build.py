"""Builds libbsscl_hip.so for gfx950 with hipcc (in-tree, next to this file).

    python -m bsscl_gbm._build          # from bsscl-gbm_amd/

Every source is compiled for gfx950 only, with packed-FP32 instructions
disabled (-packed-fp32-ops).  The host parts are plain C++17 compiled by the
same hipcc invocation.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)                      # bsscl-gbm_amd/
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(os.path.dirname(ROOT), "include")
LIB_NAME = "libbsscl_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
OBJ_DIR = os.path.join(ROOT, "_build")

SOURCES = ["kernels.hip", "fisher_yates.hip", "colsort.hip", "engine.hip", "sampler.cpp"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the engine)")


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-result",
        f"-I{INCLUDE}", f"-I{CSRC}",
    ]


def build(verbose: bool = False) -> str:
    """Compiles every source and links the shared library; returns its path."""
    cc = hipcc()
    os.makedirs(OBJ_DIR, exist_ok=True)
    objs = []
    for src in SOURCES:
        path = os.path.join(CSRC, src)
        obj = os.path.join(OBJ_DIR, src + ".o")
        # .cpp sources are host code that calls the HIP runtime only.
        lang = [] if src.endswith(".hip") else ["-x", "hip", "--offload-host-only"]
        cmd = [cc, *flags(), *lang, "-c", path, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        objs.append(obj)
    tmp = LIB_PATH + ".tmp"
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lpthread"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB_PATH)
