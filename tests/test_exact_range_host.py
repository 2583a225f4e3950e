"""The library's exact-wide proof arithmetic against unbounded integers (CPU).

tests/exact_range_check.cpp is built from rns8_amd/csrc/exact_axes.hpp, the
header the device kernels that prove exact-wide operands and admit their
products are built from (exact_axes.hip; reference src/core/exact_range.hpp
:34-157). Each case here goes through it and through oracle/exact_range.py
(Python integers, as unbounded as the reference's cpp_int).

The kernels compute in 256 bits: exactly for the summaries of 64-bit
operands and their products, saturating at 2^256 - 1 where carried summaries
make a candidate larger. So every bound and carried summary must equal
min(the unbounded value, 2^256 - 1), and every status the unbounded one.
The cases include carried summaries far above 2^128, where a wrapping 256-bit
product would be wrong: two results of bound 2^128 multiplied with k = 1 have
a bound of 2^256, which must be refused at every prefix, never wrapped to 0
and admitted.
"""
from __future__ import annotations

import random
import shutil
import subprocess
from pathlib import Path

import pytest

import oracle
from oracle import exact_range as xr

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def checker(tmp_path_factory) -> Path:
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("exact") / "exact_range_check"
    subprocess.run([gxx, "-O2", "-std=c++17", "-pthread", "-I", str(ROOT / "rns8_amd" / "csrc"), "-I",
                    str(ROOT / "include"), str(ROOT / "tests" / "exact_range_check.cpp"), "-o", str(exe)],
                   check=True)
    return exe


def _h(v: int) -> str:
    return ("-" if v < 0 else "") + format(abs(v), "x")


def _axis(a: xr.Axis) -> str:
    return " ".join([_h(a.max_magnitude), _h(a.absolute_sum), _h(a.sum), _h(a.minimum), _h(a.maximum),
                     _h(a.deviation_sum), "1" if a.sum_known else "0"])


def _encode(signed, m, n, k, product, A: xr.Operand, B: xr.Operand) -> str:
    lines = [f"case {'S' if signed else 'U'} {m} {n} {k} {_h(product)}",
             f"{_h(A.max_magnitude)} {len(A.rows)}", *(_axis(a) for a in A.rows),
             f"{_h(B.max_magnitude)} {len(B.cols)}", *(_axis(b) for b in B.cols)]
    return "\n".join(lines) + "\n"


def _run(exe, cases):
    """cases: (signed, m, n, k, product, A, B); returns the checker's
    (status, bound, rows, cols) per case."""
    text = "".join(_encode(*c) for c in cases)
    res = subprocess.run([str(exe)], input=text, capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    lines = res.stdout.split("\n")
    out, i = [], 0
    for signed, m, n, k, product, A, B in cases:
        st, bound = lines[i].split()
        i += 1
        carried = len(A.rows) == m or len(B.cols) == n
        rows, cols = [], []
        if carried:
            rows = [tuple(int(x, 16) for x in lines[i + j].split()) for j in range(m)]
            i += m
            cols = [tuple(int(x, 16) for x in lines[i + j].split()) for j in range(n)]
            i += n
        out.append((int(st), int(bound, 16), rows, cols))
    return out


SAT = (1 << 256) - 1


def _sat(v: int) -> int:
    return min(v, SAT)


def _expect(signed, m, n, k, product, A, B):
    bound, C = xr.gemm_bound(A, B, m, n, k)
    st = 0 if xr.fits(signed, bound, product) else 5  # RNS8_SUCCESS / RNS8_RANGE_ERROR
    rows = [(_sat(a.max_magnitude), _sat(a.absolute_sum)) for a in C.rows]
    cols = [(_sat(b.max_magnitude), _sat(b.absolute_sum)) for b in C.cols]
    return st, _sat(bound), rows, cols


def _check(exe, cases):
    got = _run(exe, cases)
    for case, g in zip(cases, got):
        assert g == _expect(*case), case[:5]


def _native(rng, rows, cols, lo, hi):
    return [[rng.randint(lo, hi) for _ in range(cols)] for _ in range(rows)]


def test_native_operands_match_unbounded(checker):
    """Host operands over the whole int64 / uint64 ranges, both semantics,
    every prefix from 17 to 20."""
    rng = random.Random(11)
    cases = []
    for t in range(24):
        signed = t % 2 == 0
        m, k, n = rng.randint(1, 5), rng.randint(1, 6), rng.randint(1, 5)
        lo, hi = (-(1 << 63), (1 << 63) - 1) if signed else (0, (1 << 64) - 1)
        if t % 3 == 1:  # small magnitudes: the centre and remainder candidates decide
            lo, hi = (-40, 40) if signed else (0, 80)
        A = xr.native_operand(_native(rng, m, k, lo, hi))
        B = xr.native_operand(_native(rng, k, n, lo, hi))
        cases.append((signed, m, n, k, oracle.modulus_product(17 + t % 4), A, B))
    _check(checker, cases)


def test_chained_results_above_2_128(checker):
    """C = A x B with bound 2^128 (attained: k = 4 products of 2^63 * 2^63 in
    the signed case, 2^64 - 1 unsigned), then C x C' with k = 1: the bound is
    2^256 (about 2^256 unsigned) and must be refused at prefix 20, as the
    reference's unbounded arithmetic refuses it."""
    P20 = oracle.modulus_product(20)
    for signed in (True, False):
        v = -(1 << 63) if signed else (1 << 64) - 1
        A = xr.native_operand([[v] * 4])
        B = xr.native_operand([[v]] * 4)
        bound, C = xr.gemm_bound(A, B, 1, 1, 4)
        assert xr.fits(signed, bound, P20)
        st, b2, rows, cols = _expect(signed, 1, 1, 1, P20, C, C)
        assert st == 5 and b2 >= 1 << 254
        _check(checker, [(signed, 1, 1, 4, P20, A, B), (signed, 1, 1, 1, P20, C, C)])


def test_large_carried_summaries(checker):
    """Synthetic carried summaries near the largest an admitted product can
    leave (max below P/2 < 2^155, absolute sums up to 2^218, k up to 2^62),
    against native operands and each other: every candidate product is far
    above 2^256 and the decisions must still equal the unbounded ones."""
    rng = random.Random(12)
    P = oracle.modulus_product(20)
    cases = []
    for t in range(16):
        signed = t % 2 == 0
        m, n = rng.randint(1, 4), rng.randint(1, 4)
        k = rng.choice([1, 2, 3, 1 << 31, (1 << 62) + 7])

        def carried(count, length):
            axes = []
            for _ in range(count):
                mx = rng.randint(1, P // 2 - 1) >> rng.randint(0, 150)
                axes.append(xr.Axis(max_magnitude=mx, absolute_sum=mx * rng.randint(1, length)))
            return xr.Operand(max(a.max_magnitude for a in axes), axes, axes)

        A = carried(m, k) if t % 4 != 3 else xr.native_operand(_native(rng, m, 3, -(1 << 63), (1 << 63) - 1))
        B = carried(n, k) if t % 4 != 2 else xr.native_operand(_native(rng, 3, n, -(1 << 63), (1 << 63) - 1))
        if t % 4 == 3:
            k = 3
            A.cols = []
            B = xr.Operand(B.max_magnitude, [], B.cols)
        if t % 4 == 2:
            k = 3
        cases.append((signed, m, n, k, P, A, B))
    _check(checker, cases)


def test_planted_wrap_is_detected(checker):
    """The comparison can see a wrap: with the multiplication reduced mod 2^256
    instead of saturated, the chained 2^128 case would be admitted; the
    oracle with the same planted reduction disagrees with the unbounded one,
    so equality with the unbounded oracle above is a real check."""
    P20 = oracle.modulus_product(20)
    A = xr.native_operand([[-(1 << 63)] * 4])
    B = xr.native_operand([[-(1 << 63)]] * 4)
    _, C = xr.gemm_bound(A, B, 1, 1, 4)
    wrapped = (1 * C.max_magnitude * C.max_magnitude) % (1 << 256)
    assert xr.fits(True, wrapped, P20)  # the planted mistake admits it
    assert not xr.fits(True, 1 * C.max_magnitude * C.max_magnitude, P20)


def _native_summaries(exe, signed, x):
    rows, cols = len(x), len(x[0])
    text = f"native {'S' if signed else 'U'} {rows} {cols}\n" + "\n".join(
        " ".join(_h(v) for v in row) for row in x) + "\n"
    res = subprocess.run([str(exe)], input=text, capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    lines = res.stdout.split("\n")
    parse = lambda line: tuple(int(f, 16) for f in line.split())
    return int(lines[0], 16), [parse(lines[1 + i]) for i in range(rows)], [parse(lines[1 + rows + j]) for j in range(cols)]


def _axis_tuple(a: xr.Axis):
    return (a.max_magnitude, a.absolute_sum, a.sum, a.minimum, a.maximum, a.deviation_sum, 1 if a.sum_known else 0)


@pytest.mark.parametrize("signed", [True, False])
@pytest.mark.parametrize("rows,cols", [(1, 1), (1, 7), (9, 1), (13, 40), (67, 5), (70, 130), (129, 65)])
def test_native_summaries_match_unbounded(checker, signed, rows, cols):
    """The summaries of a 64-bit operand, computed in the device passes'
    decomposition (per-tile partials of each row and column, extremes as
    maxima of biased values; more than one 64 x 64 tile in the larger cases),
    equal the unbounded ones, with the int64 / uint64 extremes placed in
    every case."""
    rng = random.Random(rows * 1000 + cols + signed)
    lo, hi = (-(1 << 63), (1 << 63) - 1) if signed else (0, (1 << 64) - 1)
    x = _native(rng, rows, cols, lo, hi)
    x[0][0] = lo
    x[-1][-1] = hi
    x[rows // 2][cols // 2] = lo if rows * cols > 2 else x[rows // 2][cols // 2]
    maximum, got_rows, got_cols = _native_summaries(checker, signed, x)
    want = xr.native_operand(x)
    assert maximum == want.max_magnitude
    assert got_rows == [_axis_tuple(a) for a in want.rows]
    assert got_cols == [_axis_tuple(a) for a in want.cols]


def test_saturating_word_arithmetic(checker):
    """sat_mul / sat_add / min / max of the kernels on operands of every limb
    count from 0 to 4 (products whose limb counts add up to 5 and 6 included,
    where the carry out of the top limb decides), against Python integers."""
    rng = random.Random(13)
    pairs = []
    for la in range(5):
        for lb in range(5):
            for _ in range(6):
                a = rng.getrandbits(64 * la) if la else 0
                b = rng.getrandbits(64 * lb) if lb else 0
                if la and rng.random() < 0.5:
                    a |= 1 << (64 * la - 1)  # top bit of the top limb set
                if lb and rng.random() < 0.5:
                    b |= (1 << (64 * lb)) - 1  # all ones
                pairs.append((a, b))
    pairs += [(SAT, 1), (SAT, 0), (1 << 128, (1 << 128) - 1), (1 << 128, 1 << 128), ((1 << 192) - 1, (1 << 64) + 1),
              (1 << 255, 2), ((1 << 255) - 1, 2), (SAT, SAT),
              # products whose only non-zero word above the low four is the top one, or the fifth
              (1 << 224, 1 << 224), (1 << 255, 1 << 193), (1 << 192, 1 << 64), (1 << 160, 1 << 96)]
    text = "".join(f"ops {_h(a)} {_h(b)}\n" for a, b in pairs)
    res = subprocess.run([str(checker)], input=text, capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    for (a, b), line in zip(pairs, res.stdout.split("\n")):
        got = [int(x, 16) for x in line.split()]
        assert got == [_sat(a * b), _sat(a + b), min(a, b), max(a, b)], (hex(a), hex(b))
