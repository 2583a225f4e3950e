"""Exact-wide magnitude proofs left on the device by device-pointer packs.

A device-pointer pack into an exact-wide matrix whose prefix admits every
64-bit value (P > 2^64, prefix 9 and up) proves its operand on the device
(per-row and per-column summaries and max |x|) without waiting for it; a
GEMM of such operands leaves its own proof there too (a snapshot of its
operands' summaries, from which its own are computed when needed). The host
decides admissions on a worst case while that case passes, and computes the
exact (refined) bound on the device when it does not, so every decision must
equal the one made on exact values (checked here against oracle/exact_range.py;
the operands are constant, so the refined and global-maximum bounds agree)
and every admitted result must export exactly:

* operands packed from device memory at prefix 20, their product exported to
  3 limbs against the brute-force product (the C4 path, never read back);
* chains D = (A x B) x E with every operand device-packed, E scaled so D's
  exact bound lands one step inside (admitted, exact D) and one step outside
  (RNS8_RANGE_ERROR) the range; the worst case fails, so the decision needs
  the device bound;
* the same chain after A is packed again with small values between the two
  GEMMs: C's proof must still be the one of the A it was computed from;
* a grouped GEMM of device-packed operands.
"""
import ctypes

import numpy as np
import pytest

import oracle
import rns8_amd as r
from oracle import exact_range as xr
from rns8_amd import hip, inputs

pytestmark = pytest.mark.gpu


def _pack_device(ctx, matrix, arr, signed):
    arr = np.ascontiguousarray(arr, dtype=np.int64 if signed else np.uint64)
    d = hip.malloc(arr.nbytes)
    try:
        hip.to_device(d, arr)
        fn = r.lib().rns8_mi355x_pack_i64_device if signed else r.lib().rns8_mi355x_pack_u64_device
        st = fn(ctx.ptr, matrix.ptr, ctypes.c_void_p(d), arr.shape[1], 0, None)
        hip.synchronize()  # the source buffer is freed next
        return st
    finally:
        hip.free(d)


def _sem(signed):
    return r.EXACT_WIDE_SIGNED if signed else r.EXACT_WIDE_UNSIGNED


def _plan(ctx, signed, m, n, k, prefix):
    return r.Plan(ctx, r.gemm_desc(_sem(signed), r.BOUND_NONE, m, n, k, max_prefix=prefix,
                                   flags=r.PLAN_FORCE_FIXED_PREFIX))


def _matrix(ctx, signed, rows, cols, prefix):
    return r.Matrix(ctx, r.matrix_desc(rows, cols, _sem(signed), r.BOUND_NONE, prefix))


def _export(ctx, plan, Cm, m, n, limbs, signed):
    out = np.zeros((m, n * limbs), dtype=np.uint64)
    fn = r.export_exact_wide_signed_limbs if signed else r.export_exact_wide_unsigned_limbs
    r.check(fn(ctx, plan, Cm, out, limbs), "export")
    return out


@pytest.mark.parametrize("signed", [True, False])
def test_device_packed_product_exports_exactly(gpu_ctx, signed):
    ctx = gpu_ctx
    m, n, k, prefix, L = 96, 80, 300, 20, 3
    if signed:
        A = inputs.full_int64(inputs.operand_seed(1301, "A"), (m, k))
        B = inputs.full_int64(inputs.operand_seed(1301, "B"), (k, n))
    else:
        A = inputs.splitmix64(inputs.operand_seed(1302, "A"), m * k).reshape(m, k)
        B = inputs.splitmix64(inputs.operand_seed(1302, "B"), k * n).reshape(k, n)
    plan = _plan(ctx, signed, m, n, k, prefix)
    Am, Bm, Cm = _matrix(ctx, signed, m, k, prefix), _matrix(ctx, signed, k, n, prefix), _matrix(ctx, signed, m, n, prefix)
    assert _pack_device(ctx, Am, A, signed) == r.SUCCESS
    assert _pack_device(ctx, Bm, B, signed) == r.SUCCESS
    ws = r.Workspace(ctx, plan)
    r.check(r.lib().rns8_mi355x_gemm_rns_async(ctx.ptr, plan.ptr, Am.ptr, Bm.ptr, Cm.ptr, ws.ptr, None), "gemm")
    out = _export(ctx, plan, Cm, m, n, L, signed)
    want = oracle.exact_gemm_i64(A, B, limbs=L) if signed else oracle.exact_gemm_u64(A, B, limbs=L)
    np.testing.assert_array_equal(out, want)


def _chain_unit(signed):
    """A, B with attained global maxima; C = A x B with k1 = 2 has every cell
    at C's bound, and D = C x E (E constant s, k2 = 2) has |D| = bound(D)."""
    if signed:
        a, b = -(1 << 62), (1 << 62) - 1
    else:
        a, b = (1 << 64) - 1, (1 << 63) + 7
    A = [[a, a]]
    B = [[b, b], [b, b]]
    return A, B


def _run_chain(ctx, signed, prefix, s, repack_small=False):
    A, B = _chain_unit(signed)
    m, k1, k2, n = 1, 2, 2, 2
    E = [[s] * n] * k2
    p1 = _plan(ctx, signed, m, k2, k1, prefix)
    p2 = _plan(ctx, signed, m, n, k2, prefix)
    Am, Bm, Cm = _matrix(ctx, signed, m, k1, prefix), _matrix(ctx, signed, k1, k2, prefix), _matrix(ctx, signed, m, k2, prefix)
    Em, Dm = _matrix(ctx, signed, k2, n, prefix), _matrix(ctx, signed, m, n, prefix)
    for M, src in ((Am, A), (Bm, B), (Em, E)):
        assert _pack_device(ctx, M, np.array(src, dtype=object).astype(np.int64 if signed else np.uint64), signed) \
            == r.SUCCESS
    ws1, ws2 = r.Workspace(ctx, p1), r.Workspace(ctx, p2)
    r.check(r.lib().rns8_mi355x_gemm_rns_async(ctx.ptr, p1.ptr, Am.ptr, Bm.ptr, Cm.ptr, ws1.ptr, None), "C = A x B")
    if repack_small:
        # A's new maximum is 1: C's proof must still come from the A it used
        assert _pack_device(ctx, Am, np.ones((m, k1), dtype=np.int64 if signed else np.uint64), signed) == r.SUCCESS
    st = r.lib().rns8_mi355x_gemm_rns_async(ctx.ptr, p2.ptr, Cm.ptr, Em.ptr, Dm.ptr, ws2.ptr, None)
    hip.synchronize()
    if st != r.SUCCESS:
        return st, None
    L = 4
    out = _export(ctx, p2, Dm, m, n, L, signed)
    return st, [oracle.limbs_to_int(out[0, L * j:L * j + L], signed) for j in range(n)]


def _oracle_chain_bound(signed, s):
    A, B = _chain_unit(signed)
    maxa = max(abs(v) for row in A for v in row)
    maxb = max(abs(v) for row in B for v in row)
    bc, C = xr.gemm_bound(xr.uniform_operand(maxa), xr.uniform_operand(maxb), 1, 2, 2)
    bd, _ = xr.gemm_bound(C, xr.uniform_operand(abs(s)), 1, 2, 2)
    return bd


@pytest.mark.parametrize("signed", [True, False])
@pytest.mark.parametrize("prefix", [17, 19])
def test_chain_threshold_reads_back_exact_maxima(gpu_ctx, signed, prefix):
    P = oracle.modulus_product(prefix)
    unit = _oracle_chain_bound(signed, 1)
    s = ((P - 1) // 2 if signed else P - 1) // unit
    assert s >= 2
    A, B = _chain_unit(signed)
    for step, want in ((0, r.SUCCESS), (1, r.RANGE_ERROR)):
        scale = s + step
        bound = _oracle_chain_bound(signed, scale)
        assert xr.fits(signed, bound, P) == (want == r.SUCCESS)
        st, D = _run_chain(gpu_ctx, signed, prefix, scale)
        assert st == want, (prefix, step)
        if D is not None:
            c = sum(int(x) * int(y) for x, y in zip(A[0], [row[0] for row in B]))
            assert D == [2 * c * scale] * 2
            assert abs(D[0]) == bound  # the bound is attained


@pytest.mark.parametrize("signed", [True, False])
def test_result_proof_survives_operand_repack(gpu_ctx, signed):
    prefix = 17
    P = oracle.modulus_product(prefix)
    unit = _oracle_chain_bound(signed, 1)
    s = ((P - 1) // 2 if signed else P - 1) // unit
    # outside the range with C's true proof; inside if C's proof followed A's repack
    st, _ = _run_chain(gpu_ctx, signed, prefix, s + 1, repack_small=True)
    assert st == r.RANGE_ERROR


@pytest.mark.parametrize("signed", [True, False])
@pytest.mark.parametrize("large_packs", [1, 2])
def test_repack_proves_only_the_new_maximum(gpu_ctx, signed, large_packs):
    """Device packs of one matrix in a row: the proof alternates between two
    sets and a pack's accumulators and maximum must start from zero, so after
    packs of the chain's large A and then of ones, C = A x B carries the
    maximum 1.
    At the scale one above the large-A threshold the chain is admitted only
    with that proof (a maximum carried over from an earlier pack would refuse
    it)."""
    ctx = gpu_ctx
    prefix = 17
    P = oracle.modulus_product(prefix)
    s = ((P - 1) // 2 if signed else P - 1) // _oracle_chain_bound(signed, 1) + 1
    A, B = _chain_unit(signed)
    maxb = max(abs(v) for row in B for v in row)
    bc, Cop = xr.gemm_bound(xr.uniform_operand(1), xr.uniform_operand(maxb), 1, 2, 2)
    bd, _ = xr.gemm_bound(Cop, xr.uniform_operand(abs(s)), 1, 2, 2)
    assert xr.fits(signed, bd, P)
    m, k1, k2, n = 1, 2, 2, 2
    dt = np.int64 if signed else np.uint64
    p1, p2 = _plan(ctx, signed, m, k2, k1, prefix), _plan(ctx, signed, m, n, k2, prefix)
    Am, Bm, Cm = _matrix(ctx, signed, m, k1, prefix), _matrix(ctx, signed, k1, k2, prefix), _matrix(ctx, signed, m, k2, prefix)
    Em, Dm = _matrix(ctx, signed, k2, n, prefix), _matrix(ctx, signed, m, n, prefix)
    for _ in range(large_packs):
        assert _pack_device(ctx, Am, np.array(A, dtype=object).astype(dt), signed) == r.SUCCESS
    assert _pack_device(ctx, Am, np.ones((m, k1), dtype=dt), signed) == r.SUCCESS
    assert _pack_device(ctx, Bm, np.array(B, dtype=object).astype(dt), signed) == r.SUCCESS
    assert _pack_device(ctx, Em, np.array([[s] * n] * k2, dtype=object).astype(dt), signed) == r.SUCCESS
    ws1, ws2 = r.Workspace(ctx, p1), r.Workspace(ctx, p2)
    r.check(r.lib().rns8_mi355x_gemm_rns_async(ctx.ptr, p1.ptr, Am.ptr, Bm.ptr, Cm.ptr, ws1.ptr, None), "C = A x B")
    st = r.lib().rns8_mi355x_gemm_rns_async(ctx.ptr, p2.ptr, Cm.ptr, Em.ptr, Dm.ptr, ws2.ptr, None)
    hip.synchronize()
    assert st == r.SUCCESS
    out = _export(ctx, p2, Dm, m, n, 4, signed)
    c = 2 * int(B[0][0])
    assert [oracle.limbs_to_int(out[0, 4 * j:4 * j + 4], signed) for j in range(n)] == [2 * c * s] * n


def test_grouped_device_packed_operands(gpu_ctx):
    ctx = gpu_ctx
    m, n, k, prefix, L, T = 64, 48, 200, 18, 3, 3
    plan = _plan(ctx, True, m, n, k, prefix)
    trip, want = [], []
    for t in range(T):
        A = inputs.full_int64(inputs.operand_seed(1400 + t, "A"), (m, k))
        B = inputs.full_int64(inputs.operand_seed(1400 + t, "B"), (k, n))
        Am, Bm, Cm = _matrix(ctx, True, m, k, prefix), _matrix(ctx, True, k, n, prefix), _matrix(ctx, True, m, n, prefix)
        assert _pack_device(ctx, Am, A, True) == r.SUCCESS
        assert _pack_device(ctx, Bm, B, True) == r.SUCCESS
        trip.append((Am, Bm, Cm, r.Workspace(ctx, plan)))
        want.append(oracle.exact_gemm_i64(A, B, limbs=L))
    r.check(r.gemm_rns_grouped(ctx, plan, trip), "grouped")
    for (_, _, Cm, _), w in zip(trip, want):
        np.testing.assert_array_equal(_export(ctx, plan, Cm, m, n, L, True), w)
