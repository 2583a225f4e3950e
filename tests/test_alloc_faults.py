"""Allocation-failure injection over the host layer (reference
tests/support/allocation_fault.cpp:18-118 with
tests/unit/test_exact_cpu_allocation_faults.cpp:247-300): every allocation
the library makes in a call is failed in turn, and each failure must come
back through the C API with nothing committed (tests/alloc_fault_check.cpp).

The device-free entries run here; the ones that need a context run on the
GPU (tests/test_gpu_alloc_faults.py)."""
import shutil
import subprocess

import pytest

import native_checks


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    return native_checks.build_alloc_fault_check(tmp_path_factory.mktemp("afc"))


def test_device_free_entries_under_allocation_faults(checker):
    res = subprocess.run([str(checker), "host"], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "PASS mode=host" in res.stdout
    # the per-tile schedule allocates; every one of its points was failed
    line = next(l for l in res.stdout.splitlines() if l.startswith("case=plan_schedule/per-tile"))
    assert int(line.split("allocation_points=")[1].split()[0]) > 0
