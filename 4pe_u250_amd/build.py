"""Build recipe for libswiftkv.so (gfx950) and the CPU oracle.

    python 4pe_u250_amd/build.py          # library, host driver, the phase-stamp diagnostic
                                          # library and the oracle (+ oracle/_ref when the
                                          # reference sources are present)

The library is compiled in-tree with hipcc for gfx950 only.  All HIP code is
built with packed-FP32 instruction selection disabled.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB = os.path.join(PKG_DIR, "libswiftkv.so")
ORACLE_DIR = os.path.join(REPO, "oracle")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Atomics with a returned value stay single-lane operations whose result
    # is waited for where it is used: the optimizer's wave-wide expansion
    # broadcasts the result at once, so the issuing wave would stall on the
    # round trip (the balanced scan's unit claims, the split arrival count).
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    # The leading kernel arguments (the step kernel's first eight: everything
    # its first loads depend on) are preloaded into SGPRs by the dispatcher,
    # so a wave issues its first vector loads without waiting on scalar loads
    # of the argument block.  Kernels whose first argument is a struct
    # preload nothing.
    "-mllvm", "-amdgpu-kernarg-preload-count=8",
]
SOURCES = ["swiftkv_kernels.hip", "swiftkv_synth.hip", "swiftkv_exact.hip", "swiftkv_capi.cpp"]
HOST_SRC = os.path.join(PKG_DIR, "host", "swiftkv_host.cpp")
HOST_BIN = os.path.join(PKG_DIR, "swiftkv_host")


def _run(cmd, cwd=None):
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; drop that line.
    lines = [ln for ln in proc.stdout.splitlines() if "packed-fp32-ops' is not a recognized feature" not in ln]
    if proc.returncode != 0:
        sys.stderr.write("\n".join(lines) + "\n")
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}")
    return "\n".join(lines)


def build_library(verbose: bool = False) -> str:
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *HIP_FLAGS, "-I", os.path.join(REPO, "include"), *srcs, "-o", tmp]
    out = _run(cmd)
    if verbose and out.strip():
        print(out)
    os.replace(tmp, LIB)
    return LIB


STAMPS_LIB = os.path.join(PKG_DIR, "libswiftkv_stamps.so")


def build_stamps(verbose: bool = False) -> str:
    """The instrumented library for phase_stamps.py: the same sources with the
    step kernel's s_memrealtime phase stamps compiled in (SWIFTKV_PHASE_STAMPS).
    Diagnostics only; the product is libswiftkv.so."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = STAMPS_LIB + ".tmp"
    out = _run([HIPCC, *HIP_FLAGS, "-DSWIFTKV_PHASE_STAMPS", "-I", os.path.join(REPO, "include"), *srcs, "-o", tmp])
    if verbose and out.strip():
        print(out)
    os.replace(tmp, STAMPS_LIB)
    return STAMPS_LIB


def build_host(verbose: bool = False) -> str:
    """The native host driver: plain C++ over the C ABI, linked against the
    library next to it (run path $ORIGIN)."""
    cxx = shutil.which("g++")
    if cxx is None:
        raise RuntimeError("g++ not found")
    tmp = HOST_BIN + ".tmp"
    out = _run([cxx, "-O2", "-std=c++17", "-Wall", "-Wextra", "-I", os.path.join(REPO, "include"), HOST_SRC,
                "-L", PKG_DIR, "-lswiftkv", "-Wl,-rpath,$ORIGIN", "-o", tmp])
    if verbose and out.strip():
        print(out)
    os.replace(tmp, HOST_BIN)
    return HOST_BIN


def build_oracle(verbose: bool = False) -> None:
    make = shutil.which("make")
    if make is None:
        raise RuntimeError("make not found")
    out = _run([make, "-s", "-B", "-C", ORACLE_DIR])
    if verbose and out.strip():
        print(out)


def main() -> int:
    build_oracle(verbose=True)
    print(build_library(verbose=True))
    print(build_host(verbose=True))
    print(build_stamps(verbose=True))
    return 0


if __name__ == "__main__":
    sys.exit(main())
