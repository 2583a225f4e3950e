"""Drop-in proof: the reference's own, unmodified callers build and link
against librns8.so.

Each reference example (examples/*.cpp and examples/downstream-cmake/*.cpp,
the latter through the C++ wrapper include/rns8/rns8.hpp) is compiled with the
include path pointing at the read-only reference tree and linked against this
repository's library; the link must resolve every rns8_* symbol the caller
uses. Runs only in the build container, where /root/reference exists.

The examples request RNS8_BACKEND_CPU_REFERENCE explicitly. This library
implements the HIP path only, so when run they must stop cleanly at context
creation with "unsupported backend" (the reference's status for an unavailable
backend, rns8.h:654-660), never crash.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
REF = Path("/root/reference")
LIB_DIR = ROOT / "rns8_amd"

pytestmark = [
    pytest.mark.skipif(not (REF / "examples").is_dir(), reason="reference examples exist only in the build container"),
    pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available"),
    pytest.mark.skipif(not (LIB_DIR / "librns8.so").exists(), reason="librns8.so not built"),
]

EXAMPLES = sorted((REF / "examples").glob("*.cpp")) + sorted((REF / "examples" / "downstream-cmake").glob("*.cpp"))


@pytest.mark.parametrize("src", EXAMPLES, ids=lambda p: p.name)
def test_reference_example_builds_and_links(src, tmp_path):
    exe = tmp_path / src.stem
    cmd = ["g++", "-std=c++17", "-O1", "-I", str(REF / "include"), "-I", str(src.parent), str(src),
           "-o", str(exe), "-L", str(LIB_DIR), "-l:librns8.so", f"-Wl,-rpath,{LIB_DIR}",
           "-Wl,-rpath-link,/opt/rocm/lib", "-Wl,--no-undefined"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    from rns8_amd import hip

    if hip.device_count() == 0:
        run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
        assert run.returncode == 1
        assert "unsupported backend" in (run.stderr + run.stdout).lower()
