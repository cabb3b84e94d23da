"""Compile the HIP engine into ``libma_attn.so`` (gfx950) with hipcc, in-tree.

Used by ``setup.py build_ext`` and ``__graft_entry__.build()``.  The library
is a plain C-ABI shared object (include/ma_attn.h); Python binds it with
ctypes, so no torch extension machinery (and no hipify step) is involved.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
SRC = os.path.join(PKG_DIR, "csrc", "ma_attn.hip")
HEADERS = [os.path.join(PKG_DIR, "csrc", h) for h in ("pattern.h", "device_common.h", "stream_kernel.h",
                                                         "block_kernel.h", "backward_kernel.h",
                                                         "tick_features.h")] + \
    [os.path.join(REPO_DIR, "include", h) for h in ("ma_attn.h", "ma_features.h")]
LIB = os.path.join(PKG_DIR, "libma_attn.so")
ARCH = os.environ.get("MA_ATTN_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libma_attn.so)")


def command(out: str = LIB) -> list:
    return [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        # packed-FP32 VALU forms are kept out of the device code on purpose
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(REPO_DIR, "include"),
        "-o", out, SRC,
    ]


def build(verbose: bool = True) -> str:
    """Always recompiles; writes atomically so a loaded library is never torn."""
    tmp = LIB + ".tmp"
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build()
