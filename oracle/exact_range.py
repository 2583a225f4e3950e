"""Exact-wide admission proofs in Python integers -- TEST INFRASTRUCTURE ONLY.

A restatement of the reference's magnitude proofs for exact-wide GEMMs
(src/core/exact_range.hpp), used by the tests as the checker of the library's
admission decisions (RNS8_SUCCESS vs RNS8_RANGE_ERROR). Python integers are
unbounded, as the reference's multiprecision integers are. Only small inputs
are meant: every function is a plain loop.

Pinned in tests/test_oracle_exact_range.py by what the mathematics fixes: every
bound is at least the true max |A x B| (brute force, chains included), and for
inputs where one of the candidate bounds is attained (constant operands,
operands alternating around a centre against a constant one, one-signed
columns against a constant row) the bound equals the true maximum.
"""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class Axis:
    """Summary of one row or column (reference rns8_exact_axis_range)."""

    max_magnitude: int = 0
    absolute_sum: int = 0
    sum: int = 0
    minimum: int = 0
    maximum: int = 0
    deviation_sum: int = 0
    sum_known: bool = False


@dataclass
class Operand:
    """What a packed exact-wide matrix carries into a GEMM: its largest
    magnitude and, when known, per-row and per-column summaries."""

    max_magnitude: int
    rows: list = field(default_factory=list)
    cols: list = field(default_factory=list)


def fits(signed: bool, bound: int, product: int) -> bool:
    """exact_range.hpp:16-18."""
    return bound >= 0 and (2 * bound < product if signed else bound < product)


def _center(a: Axis) -> int:
    """exact_range.hpp:24-26: (min + max) / 2, truncated toward zero."""
    s = a.minimum + a.maximum
    q = abs(s) // 2
    return q if s >= 0 else -q


def _deviation_max(a: Axis, c: int) -> int:
    """exact_range.hpp:28-32."""
    return max(abs(a.minimum - c), abs(a.maximum - c))


def _add(a: Axis, v: int, first: bool) -> None:
    """exact_range.hpp:34-47."""
    a.max_magnitude = max(a.max_magnitude, abs(v))
    a.absolute_sum += abs(v)
    a.sum += v
    if first:
        a.minimum = a.maximum = v
    else:
        a.minimum = min(a.minimum, v)
        a.maximum = max(a.maximum, v)
    a.sum_known = True


def native_operand(x) -> Operand:
    """exact_range.hpp:51-78: summaries of a host operand (a list of rows of
    Python integers), two linear scans."""
    rows_n, cols_n = len(x), len(x[0])
    rows = [Axis() for _ in range(rows_n)]
    cols = [Axis() for _ in range(cols_n)]
    maximum = 0
    for r in range(rows_n):
        for c in range(cols_n):
            v = int(x[r][c])
            _add(rows[r], v, c == 0)
            _add(cols[c], v, r == 0)
        maximum = max(maximum, rows[r].max_magnitude)
    for r in range(rows_n):
        rc = _center(rows[r])
        for c in range(cols_n):
            v = int(x[r][c])
            rows[r].deviation_sum += abs(v - rc)
            cols[c].deviation_sum += abs(v - _center(cols[c]))
    return Operand(maximum, rows, cols)


def uniform_operand(maximum: int) -> Operand:
    """An operand known only by its largest magnitude (no axis summaries)."""
    return Operand(maximum)


def axis_product_bound(a: Axis, b: Axis, k: int) -> int:
    """exact_range.hpp:80-99: a bound on |dot(row, column)| of length k."""
    bound = k * a.max_magnitude * b.max_magnitude
    bound = min(bound, a.absolute_sum * b.max_magnitude)
    bound = min(bound, a.max_magnitude * b.absolute_sum)
    if a.sum_known and b.sum_known:
        ca, cb = _center(a), _center(b)
        da, db = _deviation_max(a, ca), _deviation_max(b, cb)
        rem = min(k * da * db, a.deviation_sum * db, da * b.deviation_sum)
        center_term = ca * b.sum + cb * a.sum - k * ca * cb
        bound = min(bound, abs(center_term) + rem)
    return bound


def _uniform_axis(maximum: int, length: int) -> Axis:
    """exact_range.hpp:101-106."""
    return Axis(max_magnitude=maximum, absolute_sum=length * maximum)


def gemm_bound(A: Operand, B: Operand, m: int, n: int, k: int) -> tuple[int, Operand]:
    """exact_range.hpp:110-145: the output bound of C = A x B and the operand
    summary C carries into a later GEMM (largest magnitude; per-row and
    per-column max and absolute sum of the cell bounds, no signed sums)."""
    bound = k * A.max_magnitude * B.max_magnitude
    a_rows = len(A.rows) == m
    b_cols = len(B.cols) == n
    if not (a_rows or b_cols):
        return bound, Operand(bound)
    fa, fb = _uniform_axis(A.max_magnitude, k), _uniform_axis(B.max_magnitude, k)
    rows = [Axis() for _ in range(m)]
    cols = [Axis() for _ in range(n)]
    maximum = 0
    for r in range(m):
        a = A.rows[r] if a_rows else fa
        for c in range(n):
            b = B.cols[c] if b_cols else fb
            cell = axis_product_bound(a, b, k)
            maximum = max(maximum, cell)
            rows[r].max_magnitude = max(rows[r].max_magnitude, cell)
            cols[c].max_magnitude = max(cols[c].max_magnitude, cell)
            rows[r].absolute_sum += cell
            cols[c].absolute_sum += cell
    bound = min(bound, maximum)
    return bound, Operand(bound, rows, cols)


def pack_admits(signed: bool, x, product: int) -> bool:
    """Admission of one operand at pack time: its largest magnitude must fit
    the prefix's range (exact_range.hpp:16-18 applied to max |x|)."""
    return fits(signed, max(abs(int(v)) for row in x for v in row), product)
