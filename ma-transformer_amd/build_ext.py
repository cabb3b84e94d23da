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
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
# one object per translation unit, compiled in parallel, then linked
SOURCES = [os.path.join(CSRC, f) for f in ("ma_attn.hip", "encoder_layer.hip")]
LIB = os.path.join(PKG_DIR, "libma_attn.so")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
ARCH = os.environ.get("MA_ATTN_ARCH", "gfx950")

# packed-FP32 VALU forms are kept out of the device code on purpose
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libma_attn.so)")


def compile_command(src: str, obj: str) -> list:
    return [hipcc(), f"--offload-arch={ARCH}", *FLAGS, "-I", os.path.join(REPO_DIR, "include"),
            "-c", "-o", obj, src]


def link_command(objs: list, out: str = LIB) -> list:
    return [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out, *objs]


def _run(cmd: list, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(verbose: bool = True) -> str:
    """Always recompiles every translation unit (in parallel) and links;
    writes atomically so a loaded library is never torn."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    objs = [os.path.join(BUILD_DIR, os.path.basename(s) + ".o") for s in SOURCES]
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        for f in [pool.submit(_run, compile_command(s, o), verbose) for s, o in zip(SOURCES, objs)]:
            f.result()
    tmp = LIB + ".tmp"
    _run(link_command(objs, tmp), verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build()
