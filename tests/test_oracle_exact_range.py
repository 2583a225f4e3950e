"""Pins the exact-wide admission oracle (oracle/exact_range.py, a restatement of
the reference's src/core/exact_range.hpp) by what the mathematics fixes:

* soundness: every bound is at least the true max |A x B| (brute force in Python
  integers), for native operands, operands known only by their maximum, and
  chains (A x B) x E that use the summaries C carries;
* attainment: where one candidate bound is attained by the product, the bound
  is that maximum exactly:
  - constant operands: k * |a| * |b|;
  - a constant row against one-signed columns: |a| * max_j sum_k |B[k][j]|;
  - rows alternating c + d, c - d around a centre against a constant column:
    k * |c| * |e|, below the plain k * max|A| * max|B| (the centre refinement
    of exact_range.hpp:88-97 decides);
  - a constant chain: k2 * k1 * |a| * |b| * |e|;
* the admission rule: 2 * bound < P (signed), bound < P (unsigned).

A dropped candidate (of the bound or of the remainder), a sign error or swapped
sums in the centre term, a rounded-up centre or a missing remainder fails one
of them.
"""
import random

import pytest

from oracle import exact_range as xr


def _matmul(A, B):
    k, n = len(B), len(B[0])
    return [[sum(row[t] * B[t][j] for t in range(k)) for j in range(n)] for row in A]


def _maxabs(M):
    return max(abs(v) for row in M for v in row)


def _rand(rng, rows, cols, lo, hi):
    return [[rng.randint(lo, hi) for _ in range(cols)] for _ in range(rows)]


DISTS = [(-(1 << 62), (1 << 62)), (0, 1 << 40), (-5, 5), (1000, 1010), (-(1 << 63), -(1 << 63) + 50), (0, 1)]


@pytest.mark.parametrize("seed", range(40))
def test_bound_is_sound(seed):
    rng = random.Random(seed)
    m, k, n = rng.randint(1, 6), rng.randint(1, 9), rng.randint(1, 6)
    A = _rand(rng, m, k, *DISTS[seed % len(DISTS)])
    B = _rand(rng, k, n, *DISTS[(seed // 2) % len(DISTS)])
    truth = _maxabs(_matmul(A, B))
    for a_op in (xr.native_operand(A), xr.uniform_operand(_maxabs(A))):
        for b_op in (xr.native_operand(B), xr.uniform_operand(_maxabs(B))):
            bound, carried = xr.gemm_bound(a_op, b_op, m, n, k)
            assert bound >= truth
            assert carried.max_magnitude == bound
            if carried.rows:
                C = _matmul(A, B)
                for r in range(m):
                    assert carried.rows[r].max_magnitude >= max(abs(v) for v in C[r])
                    assert carried.rows[r].absolute_sum >= sum(abs(v) for v in C[r])
                for c in range(n):
                    assert carried.cols[c].max_magnitude >= max(abs(C[r][c]) for r in range(m))
                    assert carried.cols[c].absolute_sum >= sum(abs(C[r][c]) for r in range(m))
                    assert not carried.cols[c].sum_known


@pytest.mark.parametrize("seed", range(20))
def test_chain_bound_is_sound(seed):
    rng = random.Random(100 + seed)
    m, k1, k2, n = rng.randint(1, 5), rng.randint(1, 6), rng.randint(1, 6), rng.randint(1, 5)
    A = _rand(rng, m, k1, *DISTS[seed % len(DISTS)])
    B = _rand(rng, k1, k2, *DISTS[(seed + 1) % len(DISTS)])
    E = _rand(rng, k2, n, *DISTS[(seed + 2) % len(DISTS)])
    _, C_op = xr.gemm_bound(xr.native_operand(A), xr.native_operand(B), m, k2, k1)
    bound, _ = xr.gemm_bound(C_op, xr.native_operand(E), m, n, k2)
    assert bound >= _maxabs(_matmul(_matmul(A, B), E))


@pytest.mark.parametrize("a,b,k", [(3, -7, 5), (-(1 << 62), (1 << 62) - 1, 9), (0, 5, 3), (1, 1, 1)])
def test_constant_operands_attain(a, b, k):
    A, B = [[a] * k for _ in range(3)], [[b] * 4 for _ in range(k)]
    bound, _ = xr.gemm_bound(xr.native_operand(A), xr.native_operand(B), 3, 4, k)
    assert bound == k * abs(a) * abs(b) == _maxabs(_matmul(A, B))


def test_one_signed_columns_attain():
    rng = random.Random(7)
    k, n, a = 6, 5, -11
    B = _rand(rng, k, n, 1, 1 << 30)
    A = [[a] * k, [a] * k]
    bound, _ = xr.gemm_bound(xr.native_operand(A), xr.native_operand(B), 2, n, k)
    truth = abs(a) * max(sum(B[t][j] for t in range(k)) for j in range(n))
    assert bound == truth == _maxabs(_matmul(A, B))


@pytest.mark.parametrize("c,d,e,k", [(2, 5, 3, 4), (-(1 << 40), 3 << 40, 7, 6), (1, 1 << 61, -1, 2)])
def test_centre_refinement_attains(c, d, e, k):
    # rows c+d, c-d, ... (k even, d > |c|, so the entries change sign): row
    # centre c, row sum k*c; B constant e
    A = [[c + d if t % 2 == 0 else c - d for t in range(k)] for _ in range(2)]
    B = [[e] * 3 for _ in range(k)]
    bound, _ = xr.gemm_bound(xr.native_operand(A), xr.native_operand(B), 2, 3, k)
    assert bound == k * abs(c) * abs(e) == _maxabs(_matmul(A, B))
    # the magnitude and absolute-sum candidates alone would be larger
    assert bound < (k // 2) * (abs(c + d) + abs(c - d)) * abs(e)


# Row/column pairs for which exactly one candidate of exact_range.hpp:80-99
# equals |dot(a, b)| and every other candidate is larger (found by a random
# search over small vectors): absolute sum of a times max |b|; max |a| times
# absolute sum of b; the centre term with a zero remainder; the centre term
# with the remainder's deviation_sum(a) * dev_max(b) term strictly smallest;
# the same with dev_max(a) * deviation_sum(b).
UNIQUE = [([-3, 0], [6, 1], 18), ([-2, 1], [5, 0], 10), ([3, -5, -1], [-6, -6, -6], 18), ([5, -8], [4, 6], 28),
          ([2, -1], [-5, -4], 6)]


@pytest.mark.parametrize("case", range(len(UNIQUE)))
@pytest.mark.parametrize("sa,sb", [(1, 1), (1 << 30, 1 << 31), (-2, 6)])
def test_each_candidate_decides(case, sa, sb):
    a, b, truth = UNIQUE[case]
    A = [[sa * x for x in a]]
    B = [[sb * y] for y in b]
    bound, _ = xr.gemm_bound(xr.native_operand(A), xr.native_operand(B), 1, 1, len(a))
    assert bound == truth * abs(sa * sb) == _maxabs(_matmul(A, B))


def test_constant_chain_attains():
    a, b, e, k1, k2 = 7, -3, 5, 4, 6
    A, B, E = [[a] * k1] * 2, [[b] * 3] * k1, [[e] * 2] * 3
    _, C_op = xr.gemm_bound(xr.native_operand(A), xr.native_operand(B), 2, 3, k1)
    bound, _ = xr.gemm_bound(C_op, xr.native_operand(E), 2, 2, 3)
    assert bound == 3 * k1 * abs(a * b * e) == _maxabs(_matmul(_matmul(A, B), E))


def test_centre_truncates_toward_zero():
    # min + max odd and negative: the centre is -(|s| // 2), as C++ division
    axis = xr.native_operand([[-5, 2]]).rows[0]
    assert xr._center(axis) == -1
    axis = xr.native_operand([[5, -2]]).rows[0]
    assert xr._center(axis) == 1


def test_admission_rule():
    P = 65280  # 256 * 255
    assert xr.fits(True, (P - 1) // 2, P) and not xr.fits(True, P // 2, P)
    assert xr.fits(False, P - 1, P) and not xr.fits(False, P, P)
    assert not xr.fits(True, -1, P)
