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


def test_crt64_tail(checker):
    """The 64-bit CRT-basis export tail at P = 9..11 against __int128: low
    word and int64 / uint64 range decisions for ~1.08 million values per
    prefix, dense across every decision band (around +-2^62, +-2^63, 2^64
    and +-M/2) and random over the whole centered range."""
    out = _run(checker, "crt64")
    for p in (9, 10, 11):
        assert f"crt64 P{p}:" in out


def test_crt_export_address_gate(checker):
    """crt_export_fits admits exactly the exports whose output row bytes,
    lane offsets and unit count the CRT-basis kernel can form in 32 bits
    (one 8-limb row of 7e7 cells is refused)."""
    out = _run(checker, "crtgate")
    assert "crtgate checks" in out


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


# ---- CRT-basis export (rns8_amd/csrc/crt_export.hpp) ---------------------------


def _centered(x: int, m: int) -> int:
    r = x % m
    return r - m if r >= (m + 1) // 2 else r


def _crt_vectors(P: int, M: int, rng) -> list:
    """(residue vector, expected centered value) pairs: random centered
    residues, arbitrary int8 residues, and integers at the edges of the
    centered range [-M/2, M/2) and in the band 0.42 M .. 0.5 M where the
    quotient estimate can be off by one."""
    mods = LADDER[:P]
    out = []

    def add_x(x):
        out.append(([_centered(x, m) for m in mods], (x + M // 2) % M - M // 2))

    for x in (0, 1, -1, 2, -2, M // 2 - 1, -(M // 2), M // 2, -(M // 2) + 1, M // 2 - 2, (1 << 63) - 1, -(1 << 63),
              (1 << 64) - 1, 1 << 63):
        add_x(x)
    for k in range(6):
        add_x(M // 2 - 1 - k)
        add_x(-(M // 2) + k)
    for _ in range(120):
        add_x(rng.randrange(-(M // 2), M // 2))
    for _ in range(60):
        mag = rng.randrange(M * 42 // 100, M // 2)
        add_x(mag if rng.random() < 0.5 else -mag)
    for _ in range(40):
        r = [rng.randrange(-128, 128) for _ in mods]
        # the class of an arbitrary residue vector, centered
        x = 0
        for i, (ri, mi) in enumerate(zip(r, mods)):
            mi_rest = M // mi
            x += ri * mi_rest * pow(mi_rest, -1, mi)
        out.append((r, (x + M // 2) % M - M // 2))
    return out


def test_crt_export_tables_and_tail(checker):
    """The MFMA export's tables and per-cell tail (crt_export.hpp), run on the
    CPU by tables_check: the signed base-256 digits of every CRT basis
    element K_i reconstruct K_i, the quotient digits F_i are within 1/2 of
    2^14 K_i / M, M's 16-bit limbs are M, and for every prefix 1..20 the tail
    turns the column sums of a residue vector into the centered value of its
    class, checked against Python big integers on ~250 vectors per prefix
    (range edges, the off-by-one band of the quotient estimate, arbitrary
    int8 residues)."""
    import random

    rng = random.Random(77)
    vectors = []
    for P in range(1, 21):
        M = math.prod(LADDER[:P])
        vectors += [(P, r, v) for r, v in _crt_vectors(P, M, rng)]
    text = "".join(f"{P} {' '.join(map(str, r))}\n" for P, r, _ in vectors)
    res = subprocess.run([str(checker), "crt"], input=text, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-2000:]
    lines = res.stdout.split("\n")
    assert lines[-2] == "ok"
    tables, i = {}, 0
    while lines[i].startswith("table"):
        _, P, bits, digits, limbs = lines[i].split()
        P, bits, digits, limbs = int(P), int(bits), int(digits), int(limbs)
        w = [list(map(int, lines[i + 1 + t].split()[2:])) for t in range(P)]
        m16 = list(map(int, lines[i + 1 + P].split()[1:]))
        tables[P] = (bits, digits, limbs, w, m16)
        i += P + 2
    assert sorted(tables) == list(range(1, 21))
    for P, (bits, digits, limbs, w, m16) in tables.items():
        mods = LADDER[:P]
        M = math.prod(mods)
        assert bits == M.bit_length()
        assert sum(v << (16 * j) for j, v in enumerate(m16)) == M
        for t, m in enumerate(mods):
            K = (M // m) * pow(M // m, -1, m) if P > 1 else 1
            assert all(-128 <= d <= 127 for d in w[t])
            assert sum(d * 256 ** b for b, d in enumerate(w[t][:digits])) == K
            F = w[t][digits] + 256 * w[t][digits + 1]
            assert abs(F * M - (K << 14)) * 2 <= M  # |F - 2^14 K / M| <= 1/2
    outs = [ln for ln in lines[i:] if ln.startswith("v ")]
    assert len(outs) == len(vectors)
    for (P, r, want), ln in zip(vectors, outs):
        parts = ln.split()
        assert int(parts[1]) == P
        sign, limbs_out = int(parts[2]), list(map(int, parts[3:]))
        got = sum(v << (16 * j) for j, v in enumerate(limbs_out)) + sign * (1 << (16 * len(limbs_out)))
        assert got == want, (P, r)
