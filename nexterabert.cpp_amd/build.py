"""Builds libnxg.so in-tree: the gfx950 kernels (hipcc) and the host code (g++).

    python nexterabert.cpp_amd/build.py

Flags that matter for the results being the reference's bit for bit:
  -ffp-contract=off    every multiply, add and fma is the one written in the source
  -fno-fast-math       correctly rounded fp32 division, IEEE NaN/denormal behaviour
  (hipcc's defaults keep fp32 denormals on gfx950 and round divisions correctly)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OBJ = PKG / "_build"
LIB = PKG / "libnxg.so"
ARCH = "gfx950"


def _hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and Path(c).exists():
            return c
    raise FileNotFoundError("hipcc not found (set HIPCC)")


def _run(cmd, verbose):
    cmd = [str(c) for c in cmd]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build(verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    common = ["-O3", "-fPIC", "-std=c++17", "-ffp-contract=off", "-fno-fast-math",
              "-fvisibility=hidden", "-DNXG_BUILD", f"-I{INCLUDE}", f"-I{CSRC}", "-Wall"]
    hip_only = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
    _run(["g++", *common, "-pthread", "-c", CSRC / "nxg_host.cpp", "-o", OBJ / "nxg_host.o"], verbose)
    _run(["g++", *common, "-c", CSRC / "nxg_gguf.cpp", "-o", OBJ / "nxg_gguf.o"], verbose)
    _run([_hipcc(), *hip_only, *common, "-c", CSRC / "nxg_linear.hip", "-o", OBJ / "nxg_linear.o"], verbose)
    tmp = LIB.with_suffix(".so.tmp")
    _run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread",
          OBJ / "nxg_linear.o", OBJ / "nxg_host.o", OBJ / "nxg_gguf.o", "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-q" not in sys.argv[1:]))
