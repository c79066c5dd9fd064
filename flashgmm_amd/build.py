"""Builds ``flashgmm_amd/libflashgmm.so`` (hipcc, gfx950) and the host path
``flashgmm_amd/libflashgmm_cpu.so`` (g++, OpenMP) in-tree.

Usage: ``python -m flashgmm_amd.build`` (or ``__graft_entry__.build()``).
Each ``csrc/*.hip`` translation unit is compiled to an object under
``flashgmm_amd/_build/`` in parallel, then linked into one shared library
that exports the C ABI declared in ``include/flashgmm.h``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OUT = os.path.join(PKG, "libflashgmm.so")
BUILD = os.path.join(PKG, "_build")
ARCH = os.environ.get("FLASH_GMM_HIP_ARCH", "gfx950")

SOURCES = ["fgmm_api.hip", "fgmm_common.hip", "fgmm_mfma.hip", "fgmm_valu.hip", "fgmm_x32.hip",
           "fgmm_resp.hip", "fgmm_sparse.hip", "fgmm_small.hip"]

# Packed-fp32 VALU forms are disabled for all device code (the compiler would
# otherwise form v_pk_* fp32 ops from plain float code).
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall",
          "-Wno-unused-result", "-I", os.path.join(ROOT, "include")] + DEVICE_FLAGS


def hipcc() -> str:
    cand = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(cand):
        raise RuntimeError("hipcc not found (ROCm toolchain required to build libflashgmm)")
    return cand


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *COMMON, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


# The host path (CPU tensors): plain C++ with OpenMP, no HIP.  AVX2 + FMA is
# the vector baseline of every x86-64 host these boxes use.
CPU_SRC = os.path.join(CSRC, "cpu", "fgmm_cpu.cpp")
CPU_OUT = os.path.join(PKG, "libflashgmm_cpu.so")
CPU_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", "-fopenmp", "-mavx2", "-mfma", "-Wall",
             "-I", os.path.join(ROOT, "include")]


def build_cpu(verbose: bool = True) -> str:
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("g++ not found (needed for libflashgmm_cpu.so)")
    tmp = CPU_OUT + ".tmp"
    cmd = [cxx, *CPU_FLAGS, CPU_SRC, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed:\n{' '.join(cmd)}\n{r.stderr}")
    if r.stderr.strip():
        sys.stderr.write(r.stderr + "\n")
    os.replace(tmp, CPU_OUT)
    if verbose:
        print(f"[flashgmm_amd] built {CPU_OUT}")
    return CPU_OUT


def build(verbose: bool = True) -> str:
    build_cpu(verbose)
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"[flashgmm_amd] built {OUT}")
    return OUT


if __name__ == "__main__":
    build()
