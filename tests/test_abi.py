"""The drop-in boundary: librns8.so exports exactly the C ABI that include/
declares, with the reference's struct layouts and constants, and its
device-free entry points behave like the reference's (CPU only, no kernels).

Reference interface: include/rns8/{rns8.h,moduli.h,status.h,abi.h,bounds.h,
semantics.h} of the reference tree. The layout check compiles one generated
program against the reference headers and against this repository's headers
and compares every sizeof / alignof / offsetof and every enumerator and
#define constant it prints; it runs only where /root/reference exists.
"""
from __future__ import annotations

import ctypes as C
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
INCLUDE = ROOT / "include"
REF_INCLUDE = Path("/root/reference/include")
LIB_PATH = ROOT / "rns8_amd" / "librns8.so"


def declared_functions(paths) -> set[str]:
    names = set()
    for p in paths:
        text = re.sub(r"/\*.*?\*/", " ", Path(p).read_text(), flags=re.S)
        text = re.sub(r"^\s*#[^\n]*", " ", text, flags=re.M)
        for decl in re.findall(r"RNS8_API[^;]*?\(", text):
            names.add(re.findall(r"(\w+)\s*\($", decl)[0])
    return names


def exported_symbols() -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


@pytest.fixture(scope="module")
def lib():
    if not LIB_PATH.exists():
        pytest.skip("librns8.so not built (run __graft_entry__.build())")
    import rns8_amd

    return rns8_amd.lib()


def test_exports_exactly_the_declared_abi(lib):
    headers = sorted((INCLUDE / "rns8").glob("*.h")) + [INCLUDE / "rns8_mi355x.h"]
    declared = declared_functions(headers)
    exported = exported_symbols()
    assert declared, "no declarations parsed"
    assert declared - exported == set(), f"declared but not exported: {sorted(declared - exported)}"
    assert exported - declared == set(), f"exported but not declared: {sorted(exported - declared)}"


@pytest.mark.skipif(not REF_INCLUDE.is_dir(), reason="reference headers are only in the build container")
def test_reference_entry_points_all_present(lib):
    ref = declared_functions(sorted((REF_INCLUDE / "rns8").glob("*.h")))
    ours = declared_functions(sorted((INCLUDE / "rns8").glob("*.h")))
    assert ref == ours


def _struct_members(text: str) -> dict[str, list[str]]:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    out = {}
    for name, body, close in re.findall(r"typedef struct (\w+)\s*\{(.*?)\}\s*(\w+)\s*;", text, flags=re.S):
        members = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            m = re.search(r"(\w+)\s*(\[[^\]]*\])?\s*$", decl)
            if m:
                members.append(m.group(1))
        out[close] = members
    return out


def _constants(text: str) -> list[str]:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    names = re.findall(r"^\s*(RNS8_[A-Z0-9_]+)\s*=", text, flags=re.M)
    names += re.findall(r"^#define\s+(RNS8_[A-Z0-9_]+)\s+[(\w]", text, flags=re.M)
    skip = {"RNS8_API", "RNS8_ENUM_BASE"}
    return [n for n in names if n not in skip and not n.endswith("_H")]


@pytest.mark.skipif(not REF_INCLUDE.is_dir(), reason="reference headers are only in the build container")
@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_struct_layouts_and_constants_match_reference(tmp_path):
    structs, consts = {}, []
    for h in sorted((REF_INCLUDE / "rns8").glob("*.h")):
        t = h.read_text()
        structs.update(_struct_members(t))
        consts += _constants(t)
    assert "rns8_gemm_desc" in structs and len(consts) > 50
    lines = ['#include <cstddef>', '#include <cstdio>', '#include "rns8/rns8.h"', "int main() {"]
    for s, members in sorted(structs.items()):
        lines.append(f'  std::printf("{s} size %zu align %zu\\n", sizeof({s}), alignof({s}));')
        for mbr in members:
            lines.append(f'  std::printf("{s}.{mbr} %zu\\n", offsetof({s}, {mbr}));')
    for c in sorted(set(consts)):
        lines.append(f'  std::printf("{c} %lld\\n", (long long)({c}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.cpp"
    src.write_text("\n".join(lines) + "\n")
    outputs = []
    for inc in (REF_INCLUDE, INCLUDE):
        exe = tmp_path / f"layout_{len(outputs)}"
        subprocess.run(["g++", "-std=c++17", "-I", str(inc), str(src), "-o", str(exe)], check=True)
        outputs.append(subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout)
    assert outputs[0] == outputs[1]
    assert outputs[0].count(" size ") == len(structs)


def test_device_free_queries(lib):
    """moduli.h / status.h entry points need no device (moduli.cpp:10-62)."""
    from rns8_amd import abi

    lib.rns8_default_modulus_count.restype = C.c_uint32
    lib.rns8_default_modulus.restype = C.c_uint16
    lib.rns8_default_modulus.argtypes = [C.c_uint32]
    lib.rns8_prefix_range_bits.restype = C.c_double
    lib.rns8_prefix_range_bits.argtypes = [C.c_uint32]
    import oracle

    assert lib.rns8_default_modulus_count() == 28
    assert [lib.rns8_default_modulus(i) for i in range(28)] == oracle.LADDER
    assert lib.rns8_default_modulus(28) == 0
    for p in range(0, 30):
        assert lib.rns8_prefix_range_bits(p) == pytest.approx(oracle.lib().orc_prefix_range_bits(p), abs=1e-12)
    assert lib.rns8_validate_default_moduli() == abi.SUCCESS
    for code in range(0, 12):
        assert lib.rns8_status_string(code)


def test_select_prefix_matches_oracle(lib):
    """Plan prefix selection (moduli.cpp:208-387, api_plan_schedule.inc:263-278)
    against the oracle over bounds, budgets, semantics and the force flag."""
    import oracle
    import rns8_amd as r

    out = C.c_uint32(0)
    cases = 0
    for sem, bk in ((r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS), (r.BOUNDED_U64, r.BOUND_GLOBAL_MAX_UNSIGNED),
                    (r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_UNSIGNED)):
        for bound in (0, 1, 100, 1 << 40, (1 << 62), (1 << 63) - 1, 1 << 63, (1 << 64) - 1):
            for budget in (0, 1, 5, 8, 9, 12, 20, 21):
                for flags in (0, r.PLAN_FORCE_FIXED_PREFIX):
                    desc = r.gemm_desc(sem, bk, 64, 64, 4096, bound=bound, max_prefix=budget, flags=flags)
                    st, prefix = r.select_prefix(desc)
                    ost = oracle.lib().orc_select_prefix(sem, bk, bound, 4096, budget, flags, 0, 0, C.byref(out))
                    assert st == ost, (sem, bk, bound, budget, flags)
                    if st == 0:
                        assert prefix == out.value
                    cases += 1
    for lhs, rhs, k in ((1, 1, 1), (1 << 20, 1 << 20, 4096), (1 << 31, 1 << 31, 2), (1 << 40, 1 << 30, 1 << 20)):
        for sem in (r.BOUNDED_I64, r.BOUNDED_U64):
            desc = r.gemm_desc(sem, r.BOUND_INPUT_RANGE_AND_K, 8, 8, k, lhs_bound=lhs, rhs_bound=rhs)
            st, prefix = r.select_prefix(desc)
            ost = oracle.lib().orc_select_prefix(sem, r.BOUND_INPUT_RANGE_AND_K, 0, k, 0, 0, lhs, rhs,
                                                 C.byref(out))
            assert st == ost and (st != 0 or prefix == out.value)
    assert cases > 300


def test_context_without_device_reports_status(lib):
    """With no GPU visible, context creation returns a status, never crashes."""
    from rns8_amd import hip

    if hip.device_count() > 0:
        pytest.skip("a GPU is visible")
    handle = C.c_void_p()
    st = lib.rns8_create_context(0, None, C.byref(handle))
    assert st != 0 and not handle.value
    st = lib.rns8_create_context(-1, None, C.byref(handle))
    assert st != 0 and not handle.value


def test_null_and_abi_guards(lib):
    from rns8_amd import abi

    assert lib.rns8_create_context(0, None, None) == abi.INVALID_ARGUMENT
    assert lib.rns8_destroy_context(None) in (abi.SUCCESS, abi.INVALID_ARGUMENT)
    out = C.c_uint32(0)
    assert lib.rns8_mi355x_select_prefix(None, C.byref(out)) == abi.INVALID_ARGUMENT
