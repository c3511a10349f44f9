"""Builds libapeiron_hip.so (all HIP kernels + the C ABI) in-tree for gfx950.

Run ``python -m apeiron_amd.build`` (``__graft_entry__.build()`` calls it).  hipcc
cross-compiles without a GPU.  Packed FP32 instructions are disabled for every HIP
translation unit (``-packed-fp32-ops``).
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libapeiron_hip.so")
SOURCES = ["ah_gemv.hip", "ah_gemm.hip", "ah_abi.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs: the GEMM folds every MFMA result with VALU instructions,
    # and results placed in AGPRs would each need a v_accvgpr_read first
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-but-set-variable",
    "-I", os.path.join(ROOT, "include"),
]


DRIVER_SRC = os.path.join(ROOT, "tests", "cpp", "abi_driver.cpp")
DRIVER = os.path.join(ROOT, "tests", "cpp", "abi_driver")


def build_driver(out: str = DRIVER, verbose: bool = False) -> str:
    """The C++ ABI driver (tests/cpp/abi_driver.cpp): plain g++, dlopen at run time, no HIP."""
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"),
           DRIVER_SRC, "-ldl", "-o", out + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed ({r.returncode}):\n{r.stdout}{r.stderr}")
    os.replace(out + ".tmp", out)
    return out


def build(verbose: bool = False) -> str:
    srcs = []
    for s in SOURCES:
        srcs += ["-x", "hip", os.path.join(CSRC, s)]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *FLAGS, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)
    # A kernel whose host stub clang did not emit leaves an undefined __device_stub__ symbol: the
    # library would link and then fail to load.  Refuse it here.
    nm = subprocess.run(["nm", "-u", tmp], capture_output=True, text=True)
    missing = [l.split()[-1] for l in nm.stdout.splitlines() if "__device_stub__" in l]
    if missing:
        raise RuntimeError(f"kernel host stubs missing from the build: {missing}")
    os.replace(tmp, LIB)
    build_driver(verbose=verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
