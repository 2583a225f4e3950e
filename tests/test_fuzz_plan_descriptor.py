"""libFuzzer + AddressSanitizer + UndefinedBehaviorSanitizer over the
device-free planning entries rns8_mi355x_select_prefix and
rns8_mi355x_plan_schedule (tests/fuzz/fuzz_plan_descriptor.cpp; reference
tests/fuzz/rns8_fuzz_plan_descriptor.cpp), and over the pack -> GEMM ->
export contract (tests/fuzz/fuzz_export_contract.cpp): arbitrary plan and
matrix descriptors, strides, limb counts and workspaces go through the
entry points' checks, and every accepted call must hand the launchers
kernel arguments they accept and whose reach stays inside the matrices'
planes, the workspace and the caller's buffer. Both are built by
tests/fuzz/Makefile. CPU only: the library's host sources are compiled
instrumented, and no device is touched. A fixed seed and run count make
each run repeatable."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CLANG = Path("/opt/rocm/llvm/bin/clang++")
DEVICE_OBJS = [ROOT / "rns8_amd" / "_build" / f"{n}.o"
               for n in ("exact_axes", "export", "fused", "fused_skinny", "gemm", "pack", "skinny")]


@pytest.fixture(scope="module")
def fuzzer(tmp_path_factory):
    if not CLANG.is_file() or shutil.which("make") is None:
        pytest.skip("clang++ with libFuzzer or make not available")
    if not all(p.is_file() for p in DEVICE_OBJS):
        pytest.skip("library objects missing: run __graft_entry__.build()")
    out = tmp_path_factory.mktemp("fuzz")
    subprocess.run(["make", "-s", "-j8", "-C", str(ROOT / "tests" / "fuzz"), f"OUT={out}"], check=True,
                   timeout=600)
    return out


def test_plan_descriptor_fuzz(fuzzer):
    corpus = fuzzer / "corpus"
    corpus.mkdir()
    res = subprocess.run([str(fuzzer / "fuzz_plan_descriptor"), "-seed=1", "-runs=1500000", "-max_len=512",
                          "-print_final_stats=1", str(corpus)], capture_output=True, text=True, timeout=600,
                         cwd=fuzzer)
    assert res.returncode == 0, res.stderr[-4000:]
    assert "Done 1500000 runs" in res.stderr


REGRESSIONS = ROOT / "tests" / "fuzz" / "regressions"


# (tests/fuzz is not shipped to the GPU boxes, where these CPU tests are
# collected but not run)
@pytest.mark.parametrize("target", sorted(d.name for d in REGRESSIONS.iterdir() if d.is_dir())
                         if REGRESSIONS.is_dir() else [])
def test_saved_inputs(fuzzer, target):
    """Inputs that once failed a target (tests/fuzz/regressions/<target>/, the
    target's name without the fuzz_ prefix) run clean:
    plan_descriptor/padded_ld_near_int64_max.bin is a plan with n = 2^63 - 16,
    whose row pitch rounding overflowed int64 before the fix."""
    saved = sorted((REGRESSIONS / target).glob("*"))
    res = subprocess.run([str(fuzzer / f"fuzz_{target}"), *map(str, saved)], capture_output=True, text=True,
                         timeout=300, cwd=fuzzer)
    assert res.returncode == 0, res.stderr[-4000:]
    assert "runtime error" not in res.stderr


def test_export_contract_fuzz(fuzzer):
    corpus = fuzzer / "corpus_contract"
    corpus.mkdir()
    res = subprocess.run([str(fuzzer / "fuzz_export_contract"), "-seed=1", "-runs=1000000", "-max_len=512",
                          "-print_final_stats=1", str(corpus)], capture_output=True, text=True, timeout=600,
                         cwd=fuzzer)
    assert res.returncode == 0, res.stderr[-4000:]
    assert "Done 1000000 runs" in res.stderr
