"""CPU checks of the kernels' constant tables and integer reduction steps.

tests/tables_check.cpp includes rns8_amd/csrc/tables.hpp (the same header the
gfx950 kernels are built from), emulates each instruction step on the host and
compares against values computed independently (64/128-bit '%', and here
Python big integers for the Garner/CRT identities). The centering rule checked
is the reference's (src/cpu/cpu_reference.cpp:26-32: r >= (m+1)/2 -> r - m),
restated as ((x + floor(m/2)) mod m) - floor(m/2).
"""
from __future__ import annotations

import math
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LADDER = [256, 255, 253, 251, 247, 239, 233, 229, 227, 223, 217, 211, 199, 197, 193, 191, 181, 179, 173, 167]


@pytest.fixture(scope="module")
def checker(tmp_path_factory) -> Path:
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("tables") / "tables_check"
    subprocess.run([gxx, "-O2", "-std=c++17", "-I", str(ROOT / "rns8_amd" / "csrc"),
                    str(ROOT / "tests" / "tables_check.cpp"), "-o", str(exe)], check=True)
    return exe


def _run(exe: Path, mode: str) -> str:
    res = subprocess.run([str(exe), mode], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-2000:]
    assert res.stdout.rstrip().endswith("ok")
    return res.stdout


def test_quotients_exhaustive(checker):
    """24-bit reciprocal quotient over [0, s_max] and 32-bit reciprocal over
    [0, 2^21), every modulus 2..256."""
    out = _run(checker, "quot")
    assert "quot checks" in out


def test_epilogue_reduction_int32(checker):
    """int32 sums (full range and the |x| <= 2^30 + 128 the GEMM produces) ->
    packed centered int8, every modulus 2..256."""
    _run(checker, "reduce32")


def test_pack_reduction_int64(checker):
    """int64 / uint64 -> centered residue through the two-half byte dot
    products of the pack kernel, every modulus 2..256."""
    _run(checker, "pack64")


def test_unit_index_division(checker):
    """Reciprocal division of unit indices (n < 2^31) by every divisor up to
    5000, powers of two and their neighbours, 2^31 - 1 and random divisors."""
    out = _run(checker, "div")
    assert "div checks" in out


def test_export64_tail_edges(checker):
    """int64 / uint64 export tail at every prefix: values at and around 0,
    +-2^62, +-2^63, +-2^64 (incl. -2^64, whose low 64 bits are 0), +-2^65 and
    the ends of the centered range, bounds 0 .. 2^64 - 1, against __int128."""
    out = _run(checker, "export64")
    assert "export64 checks" in out


def _limbs(vals: list[int]) -> int:
    return sum(v << (24 * i) for i, v in enumerate(vals))


def test_garner_tables_and_digits(checker):
    """Garner tables for prefixes 1..20 and the export kernel's reconstruction
    (emulated from the same compile-time tables): the mixed-radix number
    sum v_i * P_i must reproduce every residue (Chinese remainder property),
    digits must be in range, Horner over the active limbs must equal it, the
    sign must follow the centered threshold ceil(P/2), the magnitude must be
    P - x or x, and the P / ceil(P/2) limbs must match the big-integer product."""
    out = _run(checker, "garner").splitlines()
    prefix = None
    cases = 0
    for line in out:
        if line.startswith("prefix "):
            prefix = int(line.split()[1])
            continue
        key, *rest = line.split(" ")
        if key == "m":
            m = [int(x) for x in rest]
            assert m == LADDER[:prefix]
            P = [math.prod(m[:i]) for i in range(prefix + 1)]
        elif key == "inv":
            inv = [int(x) for x in rest]
            for i in range(prefix):
                assert (inv[i] * P[i]) % m[i] == 1 % m[i]
        elif key == "bias":
            bias = [int(x) for x in rest]
            for i in range(prefix):
                assert bias[i] % m[i] == 0 and bias[i] >= 128 * inv[i]
        elif key == "w":
            w = [int(x) for x in rest]
            idx = 0
            for i in range(prefix):
                for j in range(i):
                    assert w[idx] == (-P[j] * inv[i]) % m[i]
                    idx += 1
        elif key == "product":
            limbs = [int(x) for x in rest]
            assert all(0 <= x < (1 << 24) for x in limbs)
            assert _limbs(limbs) == P[prefix]
        elif key == "half_ceil":
            limbs = [int(x) for x in rest]
            assert all(0 <= x < (1 << 24) for x in limbs)
            assert _limbs(limbs) == (P[prefix] + 1) // 2
        elif key == "case":
            parts = " ".join(rest).split("|")
            r = [int(x) for x in parts[0].split()]
            v = [int(x) for x in parts[1].split()]
            negative = int(parts[2]) == 1
            d = _limbs([int(x) for x in parts[3].split()])
            horner = _limbs([int(x) for x in parts[4].split()])
            x = sum(v[i] * P[i] for i in range(prefix))
            assert 0 <= x < P[prefix]
            for i in range(prefix):
                assert 0 <= v[i] < m[i]
                assert (x - r[i]) % m[i] == 0          # Chinese remainder property
            assert horner == x                          # Horner over the active limbs
            assert negative == (x >= (P[prefix] + 1) // 2)
            assert d == (P[prefix] - x if negative else x)
            cases += 1
        elif key == "ok":
            pass
    assert cases == 64 * 20
