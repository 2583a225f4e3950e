"""Allocation-failure injection over the entries that need a context: plan,
matrix, workspace and context creation, host pack and export staging,
exact-wide GEMM admission (single and grouped) and the oneshot cache, each
with every allocation it makes failed in turn (tests/alloc_fault_check.cpp);
the allocation-free GEMM entry point and the single exact-wide GEMM (whose
proofs live in memory allocated with the matrices) must make none. The checker is built by
__graft_entry__.build() into tests/_bin/."""
import subprocess

import pytest

import native_checks

pytestmark = pytest.mark.gpu


def test_context_entries_under_allocation_faults():
    exe = native_checks.built_alloc_fault_check()
    if exe is None:
        pytest.fail("tests/_bin/alloc_fault_check is missing: run __graft_entry__.build()")
    print("alloc_fault_check device", flush=True)
    res = subprocess.run([str(exe), "device"], capture_output=True, text=True, timeout=240)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "PASS mode=device" in res.stdout
    for case in ("create_plan/per-tile", "create_matrix/exact-wide", "pack_i64/exact-wide",
                 "gemm_rns_grouped/exact-wide", "gemm_i64_oneshot"):
        line = next(l for l in res.stdout.splitlines() if l.startswith(f"case={case} "))
        assert int(line.split("allocation_points=")[1].split()[0]) > 0, line
    # exact-wide admission keeps its proofs in memory allocated with the matrices
    assert "case=gemm_rns/exact-wide allocation_points=0" in res.stdout
    assert "case=gemm_rns_noalloc allocation_points=0" in res.stdout
