"""Build the native libraries in-tree (``test1_amd/lib``).

    python -m test1_amd.build

libsf_hip.so: hipcc for gfx950.  Packed-fp32 instruction selection is
disabled (``-target-feature -packed-fp32-ops``); the host pass of hipcc
warns that it does not know the feature, which is expected.
libsf_cpu.so: g++ with OpenMP; AVX-512 is selected per function at run time,
and -ffp-contract=off keeps every scalar operation a single rounding.  The
storage offload engine (worker threads, pread/pwrite) is in the same library.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib")
INCLUDE = os.path.join(ROOT, "include")

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
OFFLOAD_ARCH = "gfx950"


def _run(cmd, verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}")


def _atomic_out(path: str) -> str:
    return path + ".tmp"


def build_hip(verbose: bool = False) -> str:
    os.makedirs(LIB, exist_ok=True)
    out = os.path.join(LIB, "libsf_hip.so")
    tmp = _atomic_out(out)
    _run([HIPCC, f"--offload-arch={OFFLOAD_ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-I", INCLUDE, "-o", tmp, os.path.join(CSRC, "sf_hip.hip"), "-lhsa-runtime64"], verbose)
    os.replace(tmp, out)
    return out


def build_cpu(verbose: bool = False) -> str:
    os.makedirs(LIB, exist_ok=True)
    out = os.path.join(LIB, "libsf_cpu.so")
    tmp = _atomic_out(out)
    _run([CXX, "-O3", "-std=c++17", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-Wall",
          "-I", INCLUDE, "-o", tmp, os.path.join(CSRC, "sf_cpu_adam.cpp"), os.path.join(CSRC, "sf_io.cpp"),
          "-pthread"], verbose)
    os.replace(tmp, out)
    return out


def build_all(verbose: bool = False) -> None:
    build_hip(verbose)
    build_cpu(verbose)


if __name__ == "__main__":
    build_all(verbose=True)
