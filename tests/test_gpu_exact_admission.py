"""Exact-wide admission decisions at the range threshold, through the C ABI.

An exact-wide plan's prefix always covers K * 2^127 (signed) or K * 2^128
(unsigned), so a product of two host operands is always admitted; the
decision that can go either way is the one for a product whose operand is an
earlier result. rns8_gemm_rns admits it iff its bound fits the prefix, 2 *
bound < P (signed) or bound < P (unsigned), where the bound comes from the
per-row and per-column summaries that C = A x B carries (reference
exact_range.hpp:80-157), and those come from the candidates of
exact_axis_product_bound over A's rows and B's columns.

Each case is a chain D = (A x B) x E in which every bound is attained (checked
by brute force against the oracle's restatement, oracle/exact_range.py), with E
scaled so D's bound lands just inside and just outside the range: the library
must admit the first (and export D exactly) and refuse the second with
RNS8_RANGE_ERROR. The A x B pairs make a different candidate decide C's cell
bounds each time, so a dropped candidate, a wrong centre or a wrong remainder
in the library enlarges C's carried bound and changes a decision. Every
chain runs twice: packed from host arrays through the reference's entry
points, and packed from device memory through the device-pointer packs and
the stream entries. Both must take the reference's decisions: the operands'
summaries are computed on the device either way, and D's decision (whose
worst case k2 * bound(C) * max|E| never fits here) is the refined bound
computed on the device from C's summaries.
"""
import ctypes

import numpy as np
import pytest

import oracle
import rns8_amd as r
from oracle import exact_range as xr
from rns8_amd import hip

pytestmark = pytest.mark.gpu

# Row/column pairs where exactly one candidate of the bound equals |dot(a, b)|
# (the same pairs pin the oracle on the CPU): absolute sum of a times max |b|;
# max |a| times absolute sum of b; the centre term with a zero remainder; the
# centre term with each of the remainder's deviation-sum terms strictly
# smallest.
UNIQUE = [([-3, 0], [6, 1], 18), ([-2, 1], [5, 0], 10), ([3, -5, -1], [-6, -6, -6], 18), ([5, -8], [4, 6], 28),
          ([2, -1], [-5, -4], 6)]


def _int_matmul(A, B):
    return [[sum(int(x) * int(y) for x, y in zip(row, col)) for col in zip(*B)] for row in A]


def _maxabs(M):
    return max(abs(v) for row in M for v in row)


def _limbs(P):
    return P.bit_length() // 64 + 2


def _oracle_bound(A, B, E):
    _, C_op = xr.gemm_bound(xr.native_operand(A), xr.native_operand(B), len(A), len(B[0]), len(B))
    bound, _ = xr.gemm_bound(C_op, xr.native_operand(E), len(A), len(E[0]), len(E))
    return bound


def _pack_device(ctx, matrix, arr, signed):
    d = hip.malloc(arr.nbytes)
    try:
        hip.to_device(d, arr)
        fn = r.lib().rns8_mi355x_pack_i64_device if signed else r.lib().rns8_mi355x_pack_u64_device
        st = fn(ctx.ptr, matrix.ptr, ctypes.c_void_p(d), arr.shape[1], 0, None)
        hip.synchronize()  # the source is freed next
        return st
    finally:
        hip.free(d)


def _run_chain(ctx, A, B, E, prefix, signed, device=False):
    """Packs A, B, E at `prefix` (from host arrays through rns8_pack_*, or
    from device memory through the device-pointer packs and the stream
    entries), runs C = A x B (must be admitted) and D = C x E; returns
    (status of D, exported D or None)."""
    sem = r.EXACT_WIDE_SIGNED if signed else r.EXACT_WIDE_UNSIGNED
    bk = r.BOUND_NONE
    dt = np.int64 if signed else np.uint64
    m, k1, k2, n = len(A), len(B), len(E), len(E[0])
    flags = r.PLAN_FORCE_FIXED_PREFIX
    p1 = r.Plan(ctx, r.gemm_desc(sem, bk, m, k2, k1, max_prefix=prefix, flags=flags))
    p2 = r.Plan(ctx, r.gemm_desc(sem, bk, m, n, k2, max_prefix=prefix, flags=flags))
    mats = {name: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, bk, prefix))
            for name, rows, cols in (("A", m, k1), ("B", k1, k2), ("C", m, k2), ("E", k2, n), ("D", m, n))}
    pack = r.pack_i64 if signed else r.pack_u64
    for version, (name, src) in enumerate((("A", A), ("B", B), ("E", E)), start=1):
        arr = np.array(src, dtype=object).astype(dt)
        st = _pack_device(ctx, mats[name], arr, signed) if device else pack(ctx, mats[name], arr, version)
        r.check(st, "pack " + name)
    if device:
        ws1, ws2 = r.Workspace(ctx, p1), r.Workspace(ctx, p2)
        r.check(r.lib().rns8_mi355x_gemm_rns_async(ctx.ptr, p1.ptr, mats["A"].ptr, mats["B"].ptr, mats["C"].ptr,
                                                   ws1.ptr, None), "C = A x B")
        st = r.lib().rns8_mi355x_gemm_rns_async(ctx.ptr, p2.ptr, mats["C"].ptr, mats["E"].ptr, mats["D"].ptr,
                                                ws2.ptr, None)
        hip.synchronize()
    else:
        r.check(r.gemm_rns(ctx, p1, mats["A"], mats["B"], mats["C"], r.Workspace(ctx, p1)), "C = A x B")
        st = r.gemm_rns(ctx, p2, mats["C"], mats["E"], mats["D"], r.Workspace(ctx, p2))
    if st != r.SUCCESS:
        return st, None
    L = _limbs(oracle.modulus_product(prefix))
    out = np.zeros((m, n * L), dtype=np.uint64)
    export = r.export_exact_wide_signed_limbs if signed else r.export_exact_wide_unsigned_limbs
    r.check(export(ctx, p2, mats["D"], out, L), "export D")
    return st, [[oracle.limbs_to_int(out[i, L * j:L * j + L], signed) for j in range(n)] for i in range(m)]


def _threshold_pair(ctx, A, B, e_row, prefix, signed, device=False):
    """E = k2 copies of s * e_row with s the largest scale whose D bound still
    fits (step 0, admitted) and s + 1 (step 1, refused)."""
    P = oracle.modulus_product(prefix)
    limit = (P - 1) // 2 if signed else P - 1  # largest admitted bound
    k2 = len(B[0])
    unit = _oracle_bound(A, B, [list(e_row)] * k2)  # bound at scale 1; bounds scale linearly in s
    s = limit // unit
    assert s >= 64, "the scale step must be small against every candidate's excess"
    for step, want in ((0, r.SUCCESS), (1, r.RANGE_ERROR)):
        E = [[(s + step) * v for v in e_row]] * k2
        truth = _maxabs(_int_matmul(_int_matmul(A, B), E))
        bound = _oracle_bound(A, B, E)
        assert bound == truth
        assert xr.fits(signed, bound, P) == (want == r.SUCCESS)
        for M in (A, B, E):
            assert xr.pack_admits(signed, M, P)
        st, D = _run_chain(ctx, A, B, E, prefix, signed, device)
        assert st == want, (prefix, step, bound, P)
        if D is not None:
            assert D == _int_matmul(_int_matmul(A, B), E)


@pytest.mark.parametrize("device", [False, True])
@pytest.mark.parametrize("prefix", [17, 19, 20])
@pytest.mark.parametrize("case", range(len(UNIQUE)))
def test_signed_chain_threshold_each_candidate(gpu_ctx, prefix, case, device):
    a, b, _ = UNIQUE[case]
    sa, sb = 1 << 59, -(1 << 59)  # |entries| <= 8 * 2^59 < 2^63
    A = [[sa * x for x in a]] * 3
    B = [[sb * y, sb * y] for y in b]  # equal columns: C's rows are one-signed, so D's bound is attained
    _threshold_pair(gpu_ctx, A, B, [1, 1], prefix, True, device)


@pytest.mark.parametrize("device", [False, True])
@pytest.mark.parametrize("prefix", [18, 20])
def test_signed_chain_threshold_constant(gpu_ctx, prefix, device):
    A = [[-(1 << 62)] * 4] * 2
    B = [[(1 << 62) - 1] * 3] * 4
    _threshold_pair(gpu_ctx, A, B, [1, 1], prefix, True, device)


@pytest.mark.parametrize("device", [False, True])
@pytest.mark.parametrize("prefix", [17, 20])
def test_unsigned_chain_threshold_one_signed_columns(gpu_ctx, prefix, device):
    A = [[(1 << 63) + 5] * 4] * 2
    B = [[3 << 40, 1 << 40], [1 << 40, 2 << 40], [4 << 40, 1], [1 << 40, 9 << 40]]
    _threshold_pair(gpu_ctx, A, B, [1, 1], prefix, False, device)


@pytest.mark.parametrize("signed", [True, False])
def test_product_of_two_large_results_is_refused(gpu_ctx, signed):
    """C1 = A x B and C2 = A x B each carry the attained bound 2^128 (signed:
    four products of (-2^63)^2; unsigned: (2^64 - 1)^2 * 4 < 2^130) and are
    admitted at prefix 20. D = C1 x C2 with k = 1 has the bound C1 * C2, about
    2^256, far outside P20 (about 2^155): it must be refused with
    RNS8_RANGE_ERROR, as the reference's unbounded arithmetic refuses it (a
    256-bit product of the two bounds wraps to a small value)."""
    prefix = 20
    sem = r.EXACT_WIDE_SIGNED if signed else r.EXACT_WIDE_UNSIGNED
    bk = r.BOUND_NONE
    flags = r.PLAN_FORCE_FIXED_PREFIX
    v = -(1 << 63) if signed else (1 << 64) - 1
    dt = np.int64 if signed else np.uint64
    ctx = gpu_ctx
    p1 = r.Plan(ctx, r.gemm_desc(sem, bk, 1, 1, 4, max_prefix=prefix, flags=flags))
    p2 = r.Plan(ctx, r.gemm_desc(sem, bk, 1, 1, 1, max_prefix=prefix, flags=flags))
    A = r.Matrix(ctx, r.matrix_desc(1, 4, sem, bk, prefix))
    B = r.Matrix(ctx, r.matrix_desc(4, 1, sem, bk, prefix))
    C1 = r.Matrix(ctx, r.matrix_desc(1, 1, sem, bk, prefix))
    C2 = r.Matrix(ctx, r.matrix_desc(1, 1, sem, bk, prefix))
    D = r.Matrix(ctx, r.matrix_desc(1, 1, sem, bk, prefix))
    pack = r.pack_i64 if signed else r.pack_u64
    r.check(pack(ctx, A, np.full((1, 4), v, dtype=dt), 1), "pack A")
    r.check(pack(ctx, B, np.full((4, 1), v, dtype=dt), 2), "pack B")
    ws1 = r.Workspace(ctx, p1)
    r.check(r.gemm_rns(ctx, p1, A, B, C1, ws1), "C1 = A x B")
    r.check(r.gemm_rns(ctx, p1, A, B, C2, ws1), "C2 = A x B")
    L = _limbs(oracle.modulus_product(prefix))
    out = np.zeros((1, L), dtype=np.uint64)
    export = r.export_exact_wide_signed_limbs if signed else r.export_exact_wide_unsigned_limbs
    r.check(export(ctx, p1, C1, out, L), "export C1")
    c1 = oracle.limbs_to_int(out[0], signed)
    assert c1 == 4 * v * v
    bound = xr.gemm_bound(xr.uniform_operand(abs(c1)), xr.uniform_operand(abs(c1)), 1, 1, 1)[0]
    assert not xr.fits(signed, bound, oracle.modulus_product(prefix))
    assert r.gemm_rns(ctx, p2, C1, C2, D, r.Workspace(ctx, p2)) == r.RANGE_ERROR
