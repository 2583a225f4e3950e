"""Build librns8.so (gfx950) in-tree with hipcc.

Device code is compiled for gfx950 only, with packed-FP32 instruction
selection disabled. Objects go to rns8_amd/_build/, the shared library to
rns8_amd/librns8.so. Every call rebuilds (a build is seconds per file).
The rate probes bench.py reports beside its rooflines (the matrix-core rate,
rns8_amd/probe/mfma_probe.hip, and the HBM stream rate,
rns8_amd/probe/hbm_probe.hip) are built into their own small library,
rns8_amd/probe/librns8_probe.so; the product library does not contain them.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "rns8_amd"
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "librns8.so"
PROBE_SRCS = [PKG / "probe" / "mfma_probe.hip", PKG / "probe" / "hbm_probe.hip"]
PROBE_LIB = PKG / "probe" / "librns8_probe.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = ["-std=c++17", "-fPIC", "-fvisibility=hidden", f"-I{ROOT / 'include'}", f"-I{CSRC}"]
DEVICE_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
HOST_FLAGS = ["-O2", "-Wall", "-Wextra"]


# Per-file device flags. export.hip: its MFMA results are read by the VALU
# right away, so they are produced in VGPRs (no v_accvgpr_read per value);
# the GEMM kernels keep their accumulators in AGPRs.
FILE_FLAGS = {"export.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    if src.suffix == ".hip":
        cmd = [HIPCC, *COMMON, *DEVICE_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    else:
        cmd = [HIPCC, *COMMON, *HOST_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    ptmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-std=c++17", "-fPIC", "-shared", *DEVICE_FLAGS, *map(str, PROBE_SRCS), "-o", str(ptmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"probe build failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(ptmp, PROBE_LIB)
    if verbose:
        print(f"built {LIB} and {PROBE_LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
