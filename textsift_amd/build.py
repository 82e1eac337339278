"""Builds the gfx950 HIP library textsift_amd/lib/libpfhip.so with hipcc.

Run as ``python -m textsift_amd.build`` (also called by __graft_entry__.build()).
Objects go to textsift_amd/_build/, the library to textsift_amd/lib/.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libpfhip.so")

SOURCES = ["gemm_int4.hip", "gemm_w4.hip", "attention.hip", "kernels_misc.hip", "noalloc.hip", "runtime.cpp", "forward.cpp",
           "viterbi.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: multiplies and adds round separately unless a kernel
# calls fmaf(), as in the reference's WASM build.
# -packed-fp32-ops: no packed FP32 instructions anywhere in device code.
COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "--offload-arch=gfx950",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument", "-Wno-unused-value",
          "-I" + os.path.join(ROOT, "include")]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr[-6000:]}")
    warn = "\n".join(l for l in r.stderr.splitlines()
                     if "warning" in l and "packed-fp32-ops" not in l and "target-feature" not in l)
    if warn.strip():
        sys.stderr.write(warn + "\n")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_addon(verbose)
    return LIB


NODE_INCLUDE = os.environ.get("NODE_INCLUDE", "/usr/include/node")
ADDON = os.path.join(LIBDIR, "textsift-hip.node")


def build_addon(verbose: bool = True) -> str | None:
    """The Node-API module (csrc/hip_napi.cc -> lib/textsift-hip.node), linked
    against libpfhip.so next to it. Host code only: built with g++ against the
    Node headers; skipped (None) when they are not installed."""
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        if verbose:
            print(f"N-API module skipped: {NODE_INCLUDE}/node_api.h not found")
        return None
    tmp = ADDON + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-DNODE_GYP_MODULE_NAME=textsift_hip",
           "-I" + NODE_INCLUDE, "-I" + os.path.join(ROOT, "include"), os.path.join(CSRC, "hip_napi.cc"),
           "-L" + LIBDIR, "-lpfhip", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"N-API module build failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, ADDON)
    if verbose:
        print(f"built {ADDON}")
    return ADDON


def clean():
    shutil.rmtree(BUILD, ignore_errors=True)


if __name__ == "__main__":
    build()
