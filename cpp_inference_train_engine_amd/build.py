"""Build recipe of the HIP product library ``libmla_hip.so`` (gfx950 only) and of the
C++ host API ``libmla_host.so`` over it.

Every ``csrc/*.hip`` translation unit is compiled in parallel with hipcc into
``_build/`` and linked into ``libmla_hip.so`` next to this file (in-tree, so the
built library travels with the repository snapshot to the GPU box); ``host/mla_host.cpp``
is compiled with g++ into ``libmla_host.so`` beside it.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libmla_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CXXFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-Wall",
    "-Wno-unused-result", "-Wno-unused-command-line-argument",
    # Packed-fp32 VALU ops are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(REPO, "include"), "-I", CSRC,
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *CXXFLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed for {src}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("link of libmla_hip.so failed")
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    build_host(verbose)
    return LIB


HOST_LIB = os.path.join(PKG, "libmla_host.so")


def build_host(verbose: bool = False) -> str:
    """libmla_host.so: the C++20 host API (host/mla_host.hpp) over libmla_hip.so."""
    tmp = HOST_LIB + ".tmp"
    cmd = [os.environ.get("CXX", "g++"), "-std=c++20", "-O2", "-fPIC", "-shared", "-Wall",
           "-Wextra", "-I", os.path.join(REPO, "include"), "-I", os.path.join(PKG, "host"),
           os.path.join(PKG, "host", "mla_host.cpp"), "-L", PKG, "-lmla_hip",
           "-Wl,-rpath,$ORIGIN", "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("build of libmla_host.so failed")
    os.replace(tmp, HOST_LIB)
    if verbose:
        print("built", HOST_LIB)
    return HOST_LIB


if __name__ == "__main__":
    build(verbose=True)
