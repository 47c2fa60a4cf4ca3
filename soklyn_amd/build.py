"""Build libsoklyn_hip.so (gfx950) in-tree with hipcc, then the C++ host API
(soklyn_amd/host: libsoklyn_host.so and the soklyn_tool driver) with g++.

    python -m soklyn_amd.build          # or soklyn_amd.build.build()

Objects go to soklyn_amd/_build/, the shared libraries and the tool next to
their sources (all git-ignored; they travel with the tree).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsoklyn_hip.so")
HOST = os.path.join(HERE, "host")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
HOST_LIB = os.path.join(HOST, "libsoklyn_host.so")
HOST_TOOL = os.path.join(HOST, "soklyn_tool")
# the host API restates f32 expressions in the reference's evaluation order: no contraction
GXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wextra", "-I", INCLUDE, "-I", HOST]
SOURCES = ["gemm.hip", "elementwise.hip", "abi.hip"]
ARCH = os.environ.get("SOKLYN_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed fp32 VALU ops are left to the compiler's own choice: none are written by hand,
    # and the feature is disabled outright
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        msg = "\n".join(l for l in (p.stdout + p.stderr).splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"hipcc failed for {src}:\n{msg}")
    return obj


def build(verbose: bool = True) -> str:
    """Compile every HIP source and link libsoklyn_hip.so; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("link failed:\n" + p.stdout + p.stderr)
    os.replace(tmp, LIB)
    build_host()
    if verbose:
        print(f"[soklyn_amd] built {LIB}, {HOST_LIB}, {HOST_TOOL}", flush=True)
    return LIB


def _run(cmd, what):
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{p.stdout}{p.stderr}")


def build_host() -> None:
    """libsoklyn_host.so (the C++ host API over the C ABI) and soklyn_tool."""
    gxx = shutil.which("g++") or "g++"
    rocm_lib = "/opt/rocm/lib"
    _run([gxx, *GXX_FLAGS, "-shared", os.path.join(HOST, "soklyn.cpp"), os.path.join(HOST, "safetensors.cpp"),
          "-L", HERE, "-lsoklyn_hip",
          "-Wl,-rpath,$ORIGIN/..", f"-Wl,-rpath-link,{rocm_lib}", "-o", HOST_LIB + ".tmp"], "host library")
    os.replace(HOST_LIB + ".tmp", HOST_LIB)
    _run([gxx, *GXX_FLAGS, os.path.join(HOST, "soklyn_tool.cpp"), "-L", HOST, "-lsoklyn_host", "-L", HERE,
          "-lsoklyn_hip", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath,$ORIGIN/..", f"-Wl,-rpath-link,{rocm_lib}",
          "-o", HOST_TOOL + ".tmp"], "host tool")
    os.replace(HOST_TOOL + ".tmp", HOST_TOOL)


if __name__ == "__main__":
    build()
    sys.exit(0)
