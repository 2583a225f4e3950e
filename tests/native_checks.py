"""Host programs the tests run: built with g++ against librns8.so.

alloc_fault_check (tests/alloc_fault_check.cpp) interposes operator new and
the HIP allocation calls, so it must be its own executable. build() puts it
in tests/_bin/, where the GPU tests find it (the GPU box runs what was built
here); the CPU tests build their own copy in a temporary directory.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
BIN = ROOT / "tests" / "_bin"
LIB_DIR = ROOT / "rns8_amd"


def build_alloc_fault_check(out_dir: Path = BIN) -> Path:
    gxx = shutil.which("g++")
    if gxx is None:
        raise RuntimeError("g++ not available")
    out_dir.mkdir(parents=True, exist_ok=True)
    exe = out_dir / "alloc_fault_check"
    subprocess.run([gxx, "-O1", "-g", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-I", str(ROOT / "include"),
                    "-o", str(exe), str(ROOT / "tests" / "alloc_fault_check.cpp"), "-L", str(LIB_DIR), "-lrns8",
                    "-ldl", "-rdynamic", "-Wl,-rpath,$ORIGIN/../../rns8_amd", f"-Wl,-rpath,{LIB_DIR}"], check=True)
    return exe


def built_alloc_fault_check() -> Path | None:
    exe = BIN / "alloc_fault_check"
    return exe if exe.is_file() else None
