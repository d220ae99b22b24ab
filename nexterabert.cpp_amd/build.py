"""Builds libnxg.so in-tree: the gfx950 kernels (hipcc) and the host code (g++).

    python nexterabert.cpp_amd/build.py

Flags that matter for the results being the reference's bit for bit:
  -ffp-contract=off    every multiply, add and fma is the one written in the source
  -fno-fast-math       correctly rounded fp32 division, IEEE NaN/denormal behaviour
  (hipcc's defaults keep fp32 denormals on gfx950 and round divisions correctly)

The build fails if any kernel spills to scratch memory: the large GEMMs wait for their
LDS-DMA loads with constant vmcnt counts, which a spill reload (itself a vector memory
load) would silently invalidate. The per-kernel resource report is kept in
_build/kernel_resources.txt.
"""
from __future__ import annotations

import os
import re
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
# the reference's public C API (include/nexterabert.h) over libnxg.so, under the library name the
# reference's binding and CLI link against
API_LIB = PKG / "libnexterabert.so"
CLI = PKG / "nxg-cli"
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


def _check_resources(stderr: str) -> str:
    """Per-kernel VGPRs / scratch from -Rpass-analysis=kernel-resource-usage; raises if a
    kernel uses scratch memory."""
    rows, name = [], None
    for line in stderr.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            rows.append({"name": name})
            continue
        m = re.search(r"remark:\s+(VGPRs|AGPRs|ScratchSize \[bytes/lane\]|VGPRs Spill|LDS Size \[bytes/block\]|"
                      r"Occupancy \[waves/SIMD\]): (\d+)", line)
        if m and rows:
            rows[-1][m.group(1)] = int(m.group(2))
    report = "\n".join(f"{r['name']}: VGPRs {r.get('VGPRs')} AGPRs {r.get('AGPRs')} "
                        f"scratch {r.get('ScratchSize [bytes/lane]')} spill {r.get('VGPRs Spill')} "
                        f"LDS {r.get('LDS Size [bytes/block]')} occupancy {r.get('Occupancy [waves/SIMD]')}"
                        for r in rows)
    bad = [r["name"] for r in rows if r.get("ScratchSize [bytes/lane]", 0) or r.get("VGPRs Spill", 0)]
    if not rows:
        raise RuntimeError("no kernel resource report from hipcc")
    if bad:
        raise RuntimeError("kernels spill to scratch memory (breaks the GEMMs' constant vmcnt waits): " + ", ".join(bad))
    return report


def build(verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    common = ["-O3", "-fPIC", "-std=c++17", "-ffp-contract=off", "-fno-fast-math",
              "-fvisibility=hidden", "-DNXG_BUILD", f"-I{INCLUDE}", f"-I{CSRC}", "-Wall"]
    hip_only = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
    _run(["g++", *common, "-pthread", "-c", CSRC / "nxg_host.cpp", "-o", OBJ / "nxg_host.o"], verbose)
    _run(["g++", *common, "-c", CSRC / "nxg_gguf.cpp", "-o", OBJ / "nxg_gguf.o"], verbose)
    rocm = Path(_hipcc()).resolve().parent.parent
    _run(["g++", *common, "-D__HIP_PLATFORM_AMD__", f"-I{rocm / 'include'}", "-c", CSRC / "nxg_encoder.cpp",
          "-o", OBJ / "nxg_encoder.o"], verbose)
    cmd = [str(c) for c in (_hipcc(), *hip_only, *common, "-Rpass-analysis=kernel-resource-usage",
                            "-c", CSRC / "nxg_linear.hip", "-o", OBJ / "nxg_linear.o")]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stderr=subprocess.PIPE, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stderr)
        raise subprocess.CalledProcessError(r.returncode, cmd)
    (OBJ / "kernel_resources.txt").write_text(_check_resources(r.stderr) + "\n")
    tmp = LIB.with_suffix(".so.tmp")
    _run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread",
          OBJ / "nxg_linear.o", OBJ / "nxg_host.o", OBJ / "nxg_gguf.o", OBJ / "nxg_encoder.o", "-o", tmp], verbose)
    os.replace(tmp, LIB)
    tmp = API_LIB.with_suffix(".so.tmp")
    _run(["g++", "-O2", "-fPIC", "-std=c++17", "-Wall", "-fvisibility=hidden", "-DNEXTERA_SHARED", "-DNEXTERA_BUILD",
          "-D__HIP_PLATFORM_AMD__", f"-I{INCLUDE}", f"-I{rocm / 'include'}", "-shared", CSRC / "nexterabert_api.cpp",
          "-o", tmp, f"-L{PKG}", "-lnxg", f"-L{rocm / 'lib'}", "-lamdhip64", "-Wl,-rpath,$ORIGIN",
          f"-Wl,-rpath,{rocm / 'lib'}"], verbose)
    os.replace(tmp, API_LIB)
    # the C++ driver over the C ABI (nxg-cli: --info, --bench), linked against libnxg.so
    _run(["g++", "-O2", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__", f"-I{INCLUDE}", f"-I{rocm / 'include'}",
          CSRC / "nxg_cli.cpp", "-o", CLI, f"-L{PKG}", "-lnxg", f"-L{rocm / 'lib'}", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{rocm / 'lib'}"], verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-q" not in sys.argv[1:]))
