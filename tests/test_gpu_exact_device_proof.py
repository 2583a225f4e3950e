"""Exact-wide magnitude proofs computed on the device, through the C ABI.

Packs of exact-wide matrices compute the reference's per-row and per-column
summaries on the GPU (reference exact_range.hpp:34-78); GEMM results carry
the maxima and sums of their cell bounds (exact_range.hpp:80-171), computed
when a decision or rns8_mi355x_get_exact_proof needs them. Each test reads
the proofs back with rns8_mi355x_get_exact_proof and compares them field by
field with oracle/exact_range.py (Python integers), and checks the decisions
the library takes with them against the same oracle:

* native summaries of device-pointer and host-array packs, int64 and uint64
  over the full ranges with the extremes placed, strided sources, shapes of
  one to several 64 x 64 tiles with ragged edges, and prefixes above and
  below 9 (where the pack reads max |x| back before writing); and 4100 x
  2050 and 140000 x 8 operands, whose tiles run two tile rows per block and
  whose finishing launch strides over its axes (checked against numpy, in a
  range where int64 is exact);
* the carried summaries of a product, computed lazily from the snapshot of
  its operands' summaries, also over 33000 rows (more rows than waves);
* decisions at the range threshold that the worst case k * maxA * maxB
  cannot take (it is refused on both sides): chained GEMMs whose operand is a
  lazy result, grouped GEMMs and exports, with the operand scaled to the
  largest value the refined bound admits (the result exported exactly
  against the brute-force product) and one step more (refused, a refused
  group leaving every result's earlier proof and planes in place).

(A product of two packed operands is always admitted on its worst case: an
exact-wide plan's prefix must cover k * 2^127, or k * 2^128 unsigned.)
"""
import ctypes

import numpy as np
import pytest

import oracle
import rns8_amd as r
from oracle import exact_range as xr
from rns8_amd import hip, inputs

pytestmark = pytest.mark.gpu

FIELDS = ("max_magnitude", "absolute_sum", "sum", "minimum", "maximum", "deviation_sum")


def _sem(signed):
    return r.EXACT_WIDE_SIGNED if signed else r.EXACT_WIDE_UNSIGNED


def _matrix(ctx, signed, rows, cols, prefix):
    return r.Matrix(ctx, r.matrix_desc(rows, cols, _sem(signed), r.BOUND_NONE, prefix))


def _plan(ctx, signed, m, n, k, prefix):
    return r.Plan(ctx, r.gemm_desc(_sem(signed), r.BOUND_NONE, m, n, k, max_prefix=prefix,
                                   flags=r.PLAN_FORCE_FIXED_PREFIX))


def _dtype(signed):
    return np.int64 if signed else np.uint64


def _pack(ctx, matrix, x, signed, device, ld=None, version=1):
    """Packs the int list-of-lists / array x, from device memory (row stride
    ld >= cols elements) or from host memory."""
    arr = np.array(x, dtype=object).astype(_dtype(signed)) if not isinstance(x, np.ndarray) else x
    rows, cols = arr.shape
    if not device:
        fn = r.pack_i64 if signed else r.pack_u64
        return fn(ctx, matrix, arr, version)
    ld = ld or cols
    staged = np.zeros((rows, ld), dtype=arr.dtype)
    staged[:, :cols] = arr
    d = hip.malloc(staged.nbytes)
    try:
        hip.to_device(d, staged)
        fn = r.lib().rns8_mi355x_pack_i64_device if signed else r.lib().rns8_mi355x_pack_u64_device
        st = fn(ctx.ptr, matrix.ptr, ctypes.c_void_p(d), ld, 0, None)
        hip.synchronize()  # the source is freed next
        return st
    finally:
        hip.free(d)


def _axes_equal(got, want, fields):
    assert len(got) == len(want)
    for i, (g, w) in enumerate(zip(got, want)):
        for f in fields:
            assert g[f] == getattr(w, f), (i, f, g[f], getattr(w, f))


def _ints(arr):
    return [[int(v) for v in row] for row in arr]


def _random(seed, shape, signed, lo_hi=None):
    rng = np.random.default_rng(seed)
    if lo_hi is None:
        x = inputs.splitmix64(seed, shape[0] * shape[1]).reshape(shape)
        return x.view(np.int64) if signed else x
    lo, hi = lo_hi
    return rng.integers(lo, hi, size=shape, dtype=_dtype(signed), endpoint=True)


@pytest.mark.parametrize("signed", [True, False])
@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("shape,ld_pad", [((1, 1), 0), ((3, 70), 5), ((70, 3), 1), ((129, 65), 0),
                                          ((200, 300), 3)])
def test_native_summaries(gpu_ctx, signed, device, shape, ld_pad):
    ctx = gpu_ctx
    rows, cols = shape
    x = _random(1500 + rows * 7 + cols, shape, signed)
    lo, hi = (np.iinfo(np.int64).min, np.iinfo(np.int64).max) if signed else (0, np.iinfo(np.uint64).max)
    x[0, 0] = lo
    x[-1, -1] = hi
    x[rows // 2, cols // 2] = lo
    M = _matrix(ctx, signed, rows, cols, 20)
    assert _pack(ctx, M, x, signed, device, ld=cols + ld_pad if device else None) == r.SUCCESS
    bound, kind, R, C = M.exact_proof(ctx)
    want = xr.native_operand(_ints(x))
    assert kind == r.EXACT_AXES_NATIVE
    assert bound == want.max_magnitude
    _axes_equal(R, want.rows, FIELDS)
    _axes_equal(C, want.cols, FIELDS)


@pytest.mark.parametrize("signed", [True, False])
def test_native_summaries_two_tiles_per_block(gpu_ctx, signed):
    """Operands of at least 2048 tiles of 64 x 64 run the summary passes with
    two tile rows per block, the second one's elements loaded into registers
    while the first is summarized: 4100 x 2050 (65 x 33 tiles, an odd count
    of tile rows, ragged last tiles) packed from a strided device source.
    Values below 2^40 in magnitude keep the expected summaries exact in int64
    (numpy); the full-range 128-bit sums are checked on the smaller shapes."""
    rows, cols = 4100, 2050
    rng = np.random.default_rng(77 + signed)
    lo, hi = (-(1 << 40) + 1, (1 << 40) - 1) if signed else (0, (1 << 40) - 1)
    x = rng.integers(lo, hi, size=(rows, cols), dtype=np.int64, endpoint=True)
    # extremes at tile boundaries and in the last, ragged tiles
    x[0, 0], x[63, 64], x[64, 63], x[-1, -1], x[4096, 2048] = lo, hi, lo, hi, lo
    M = _matrix(gpu_ctx, signed, rows, cols, 20)
    assert _pack(gpu_ctx, M, x if signed else x.astype(np.uint64), signed, True, ld=cols + 3) == r.SUCCESS
    bound, kind, R, C = M.exact_proof(gpu_ctx)
    assert kind == r.EXACT_AXES_NATIVE
    assert bound == int(np.abs(x).max())
    for axis, got in ((1, R), (0, C)):
        want = _numpy_summaries(x, axis)
        assert len(got) == len(want["sum"])
        for f, w in want.items():
            g = np.array([a[f] for a in got], dtype=object)
            assert (g == w.astype(object)).all(), (axis, f)


def _numpy_summaries(x, axis):
    """The per-axis summaries of an int64 array whose sums stay in int64."""
    mn, mx = x.min(axis=axis), x.max(axis=axis)
    s = mn + mx
    centre = np.expand_dims((s + (s < 0)) >> 1, axis)  # truncated toward zero
    return {"max_magnitude": np.abs(x).max(axis=axis), "absolute_sum": np.abs(x).sum(axis=axis),
            "sum": x.sum(axis=axis), "minimum": mn, "maximum": mx, "deviation_sum": np.abs(x - centre).sum(axis=axis)}


@pytest.mark.parametrize("signed", [True, False])
def test_proof_launches_past_one_grid(gpu_ctx, signed):
    """Launch shapes whose grids stride: the finishing launch over more than
    131072 axes (a 140000 x 8 operand, whose 2188 tile rows also run two per
    block), and the product summaries over more than 32768 rows (a 33000 x 2
    result, against the oracle's cell bounds)."""
    ctx = gpu_ctx
    lo, hi = (-(1 << 30) + 1, (1 << 30) - 1) if signed else (0, (1 << 30) - 1)
    rng = np.random.default_rng(91 + signed)
    x = rng.integers(lo, hi, size=(140000, 8), dtype=np.int64, endpoint=True)
    x[0, 0], x[-1, -1], x[70000, 3] = lo, hi, hi
    M = _matrix(ctx, signed, *x.shape, 20)
    assert _pack(ctx, M, x if signed else x.astype(np.uint64), signed, True) == r.SUCCESS
    bound, kind, R, C = M.exact_proof(ctx)
    assert kind == r.EXACT_AXES_NATIVE and bound == int(np.abs(x).max())
    for axis, got in ((1, R), (0, C)):
        for f, w in _numpy_summaries(x, axis).items():
            assert (np.array([a[f] for a in got], dtype=object) == w.astype(object)).all(), (axis, f)

    m, k, n, prefix = 33000, 8, 2, 20
    A = [[int(v) for v in row] for row in rng.integers(lo, hi, size=(m, k), dtype=np.int64, endpoint=True)]
    B = [[int(v) for v in row] for row in rng.integers(lo, hi, size=(k, n), dtype=np.int64, endpoint=True)]
    Am, Bm, Cm = _matrix(ctx, signed, m, k, prefix), _matrix(ctx, signed, k, n, prefix), _matrix(ctx, signed, m, n, prefix)
    assert _pack(ctx, Am, A, signed, True) == r.SUCCESS
    assert _pack(ctx, Bm, B, signed, True) == r.SUCCESS
    plan = _plan(ctx, signed, m, n, k, prefix)
    r.check(_async_gemm(ctx, plan, Am, Bm, Cm, r.Workspace(ctx, plan)), "gemm")
    bound, kind, R, C = Cm.exact_proof(ctx)
    want_bound, want = xr.gemm_bound(xr.native_operand(A), xr.native_operand(B), m, n, k)
    assert kind == r.EXACT_AXES_CARRIED
    assert bound == want_bound
    _axes_equal(R, want.rows, ("max_magnitude", "absolute_sum"))
    _axes_equal(C, want.cols, ("max_magnitude", "absolute_sum"))


@pytest.mark.parametrize("signed", [True, False])
@pytest.mark.parametrize("device", [True, False])
def test_native_summaries_small_prefix(gpu_ctx, signed, device):
    """Prefix 6 (P < 2^64): the pack reads max |x| back and admits it first;
    a later pack whose maximum does not fit is refused and leaves the proof
    (and the planes) of the first."""
    ctx = gpu_ctx
    prefix = 6
    P = oracle.modulus_product(prefix)
    vmax = (P - 1) // 2 if signed else P - 1
    lo_hi = (-vmax, vmax) if signed else (0, vmax)
    x = _random(1601, (40, 90), signed, lo_hi)
    M = _matrix(ctx, signed, 40, 90, prefix)
    assert _pack(ctx, M, x, signed, device) == r.SUCCESS
    want = xr.native_operand(_ints(x))
    before = M.exact_proof(ctx)
    assert before[0] == want.max_magnitude
    _axes_equal(before[2], want.rows, FIELDS)
    _axes_equal(before[3], want.cols, FIELDS)
    planes = M.read_residues()
    y = x.copy()
    y[3, 4] = vmax + 1
    assert _pack(ctx, M, y, signed, device, version=2) == r.RANGE_ERROR
    assert M.exact_proof(ctx)[0] == before[0]
    assert M.exact_proof(ctx)[2] == before[2]
    np.testing.assert_array_equal(M.read_residues(), planes)


def _int_matmul(A, B):
    return [[sum(x * y for x, y in zip(row, col)) for col in zip(*B)] for row in A]


def _export(ctx, plan, Cm, m, n, signed, prefix):
    L = oracle.modulus_product(prefix).bit_length() // 64 + 2
    out = np.zeros((m, n * L), dtype=np.uint64)
    fn = r.export_exact_wide_signed_limbs if signed else r.export_exact_wide_unsigned_limbs
    st = fn(ctx, plan, Cm, out, L)
    if st != r.SUCCESS:
        return st, None
    return st, [[oracle.limbs_to_int(out[i, L * j:L * j + L], signed) for j in range(n)] for i in range(m)]


def _limit(signed, prefix):
    """The largest bound admitted at `prefix` (exact_range.hpp:16-18)."""
    P = oracle.modulus_product(prefix)
    return (P - 1) // 2 if signed else P - 1


def _threshold(bound_at, limit, t_max):
    """Largest scale t in [1, t_max) with bound_at(t) <= limit (bound_at is
    nondecreasing and close to linear): the bound is admitted at t and
    refused at t + 1. Bracketed around the linear estimate, then bisected."""
    t = min(max(1, limit // bound_at(1)), t_max - 1)
    d = 64
    lo, hi = max(1, t - d), min(t_max, t + d)
    while bound_at(lo) > limit:
        assert lo > 1
        lo = max(1, lo - 2 * (t - lo) - d)
    while bound_at(hi) <= limit:
        assert hi < t_max
        hi = min(t_max, hi + 2 * (hi - t) + d)
    while hi - lo > 1:
        mid = (lo + hi) // 2
        if bound_at(mid) <= limit:
            lo = mid
        else:
            hi = mid
    return lo


def _large_operands(seed, m, k, n, signed):
    """A x B whose refined bound is far below k maxA maxB. Signed: A's rows
    +-2^62 plus noise below 2^40 in magnitude (every third row negative), B's
    columns pairs (v, -v) below 2^40 in a random order (column sums and
    centres 0, so the deviation remainder decides). Unsigned: one entry 2^62
    per row of A, the rest below 2^20, B below 2^40 (A's absolute sum times
    max B decides)."""
    rng = np.random.default_rng(seed)
    if signed:
        A = [[(1 << 62) + int(v) for v in row] for row in rng.integers(-(1 << 40), 1 << 40, size=(m, k))]
        for i in range(0, m, 3):
            A[i] = [-v for v in A[i]]
        half = rng.integers(-(1 << 40), 1 << 40, size=(k // 2, n))
        B = np.concatenate([half, -half])
        for c in range(n):
            B[:, c] = B[rng.permutation(2 * (k // 2)), c]
        return A, _ints(B)
    A = rng.integers(0, 1 << 20, size=(m, k), dtype=np.uint64)
    A[np.arange(m), rng.integers(0, k, size=m)] = np.uint64(1 << 62)
    return _ints(A), _ints(rng.integers(0, 1 << 40, size=(k, n), dtype=np.uint64))


def _async_gemm(ctx, plan, A, B, C, ws):
    return r.lib().rns8_mi355x_gemm_rns_async(ctx.ptr, plan.ptr, A.ptr, B.ptr, C.ptr, ws.ptr, None)


@pytest.mark.parametrize("signed", [True, False])
def test_product_summaries_are_the_reference_ones(gpu_ctx, signed):
    ctx = gpu_ctx
    m, k, n, prefix = 23, 1024, 19, 20
    A, B = _large_operands(1700 + signed, m, k, n, signed)
    Am, Bm, Cm = _matrix(ctx, signed, m, k, prefix), _matrix(ctx, signed, k, n, prefix), _matrix(ctx, signed, m, n, prefix)
    assert _pack(ctx, Am, A, signed, True) == r.SUCCESS
    assert _pack(ctx, Bm, B, signed, True) == r.SUCCESS
    plan = _plan(ctx, signed, m, n, k, prefix)
    r.check(_async_gemm(ctx, plan, Am, Bm, Cm, r.Workspace(ctx, plan)), "gemm")
    bound, kind, R, C = Cm.exact_proof(ctx)
    a_op, b_op = xr.native_operand(A), xr.native_operand(B)
    want_bound, want = xr.gemm_bound(a_op, b_op, m, n, k)
    assert kind == r.EXACT_AXES_CARRIED
    assert bound == want_bound
    assert bound << 9 < k * a_op.max_magnitude * b_op.max_magnitude
    _axes_equal(R, want.rows, ("max_magnitude", "absolute_sum"))
    _axes_equal(C, want.cols, ("max_magnitude", "absolute_sum"))


@pytest.mark.parametrize("signed", [True, False])
@pytest.mark.parametrize("prefix", [17, 20])
@pytest.mark.parametrize("device", [True, False])
def test_chain_threshold_on_the_refined_bound(gpu_ctx, signed, prefix, device):
    """C = A x B at prefix 20 (admitted on its worst case: C's proof stays a
    lazy snapshot), then D = C x E, E = t e, at the largest scale t whose D
    bound fits `prefix` and at t + 1. The worst case k2 (k1 maxA maxB) maxE
    is refused at both, so the library computes C's summaries and D's cell
    bounds on the device, and must admit the first (D exact) and refuse the
    second."""
    ctx = gpu_ctx
    m, k1, k2, n = 9, 1024, 11, 7
    A, B = _large_operands(1900 + signed, m, k1, k2, signed)
    e = _ints(np.random.default_rng(1950).integers(1, 3, size=(k2, n), endpoint=True))
    bc, c_op = xr.gemm_bound(xr.native_operand(A), xr.native_operand(B), m, k2, k1)
    worst_c = k1 * xr.native_operand(A).max_magnitude * xr.native_operand(B).max_magnitude
    scaled = lambda t: [[t * v for v in row] for row in e]
    bound_at = lambda t: xr.gemm_bound(c_op, xr.native_operand(scaled(t)), m, n, k2)[0]
    limit = _limit(signed, prefix)
    T = _threshold(bound_at, limit, (1 << 61) if signed else (1 << 62))
    C_true = _int_matmul(A, B)
    for t, want in ((T, r.SUCCESS), (T + 1, r.RANGE_ERROR)):
        E = scaled(t)
        assert k2 * worst_c * max(v for row in E for v in row) > limit  # the worst case is refused
        Am, Bm, Cm = _matrix(ctx, signed, m, k1, 20), _matrix(ctx, signed, k1, k2, 20), _matrix(ctx, signed, m, k2, 20)
        Em, Dm = _matrix(ctx, signed, k2, n, 20), _matrix(ctx, signed, m, n, 20)
        for M, src in ((Am, A), (Bm, B), (Em, E)):
            assert _pack(ctx, M, src, signed, device) == r.SUCCESS
        p1, p2 = _plan(ctx, signed, m, k2, k1, 20), _plan(ctx, signed, m, n, k2, prefix)
        r.check(_async_gemm(ctx, p1, Am, Bm, Cm, r.Workspace(ctx, p1)), "C = A x B")
        st = _async_gemm(ctx, p2, Cm, Em, Dm, r.Workspace(ctx, p2))
        hip.synchronize()
        assert st == want, (t, bound_at(t), limit)
        assert Cm.exact_proof(ctx)[0] == bc
        if st == r.SUCCESS:
            assert Dm.exact_proof(ctx)[0] == bound_at(t)
            st, D = _export(ctx, p2, Dm, m, n, signed, prefix)
            assert st == r.SUCCESS and D == _int_matmul(C_true, E)


@pytest.mark.parametrize("signed", [True, False])
@pytest.mark.parametrize("k", [1024, 4096])
def test_export_decides_on_the_refined_bound(gpu_ctx, signed, k):
    """C = A x (t b) at prefix 20 stays lazy; exported under a plan of prefix
    17, whose range refuses C's worst case k maxA maxB, the export computes
    C's own bound and admits C at the largest t whose bound fits, and refuses
    it at t + 1. (A product of 64-bit operands is below k 2^128, so 17 is the
    one prefix of an export plan where its bound can fall either way.)"""
    ctx = gpu_ctx
    prefix = 17
    m, n = 16, 12
    rng = np.random.default_rng(2000 + signed)
    if signed:
        A = [[(1 << 62) + int(v) for v in row] for row in rng.integers(-(1 << 61), 1 << 61, size=(m, k))]
        half = rng.integers(-3, 3, size=(k // 2, n), endpoint=True)
        b = np.concatenate([half, -half])
    else:
        A = rng.integers(0, 1 << 61, size=(m, k), dtype=np.uint64)
        A[np.arange(m), rng.integers(0, k, size=m)] = np.uint64(1 << 63)
        b = rng.integers(0, 3, size=(k, n), endpoint=True)
    A, b = _ints(A), _ints(b)
    a_op = xr.native_operand(A)
    scaled = lambda t: [[t * v for v in row] for row in b]
    bound_at = lambda t: xr.gemm_bound(a_op, xr.native_operand(scaled(t)), m, n, k)[0]
    limit = _limit(signed, prefix)
    T = _threshold(bound_at, limit, 1 << 61)
    for t, want in ((T, r.SUCCESS), (T + 1, r.RANGE_ERROR)):
        B = scaled(t)
        assert k * a_op.max_magnitude * max(abs(v) for row in B for v in row) > limit
        Am, Bm, Cm = _matrix(ctx, signed, m, k, 20), _matrix(ctx, signed, k, n, 20), _matrix(ctx, signed, m, n, 20)
        assert _pack(ctx, Am, A, signed, True) == r.SUCCESS
        assert _pack(ctx, Bm, B, signed, True) == r.SUCCESS
        p20 = _plan(ctx, signed, m, n, k, 20)
        r.check(_async_gemm(ctx, p20, Am, Bm, Cm, r.Workspace(ctx, p20)), "gemm")
        hip.synchronize()
        st, C = _export(ctx, _plan(ctx, signed, m, n, 1, prefix), Cm, m, n, signed, prefix)
        assert st == want, (t, bound_at(t), limit)
        if C is not None:
            assert C == _int_matmul(A, B)


def test_grouped_refined_admission(gpu_ctx):
    """Two chain tasks D_i = C_i x E (C_i lazy results of their own A_i x B_i)
    in one group at prefix 18: admitted at the largest scale of E both bounds
    fit (each D_i exact); at one scale more the task with the smaller
    threshold is refused, so the group is refused and neither D_i's proof nor
    its planes change."""
    ctx = gpu_ctx
    signed, prefix = True, 18
    m, k1, k2, n = 8, 1024, 10, 6
    e = _ints(np.random.default_rng(2150).integers(1, 3, size=(k2, n), endpoint=True))
    scaled = lambda t: [[t * v for v in row] for row in e]
    limit = _limit(signed, prefix)
    tasks = []
    for i in range(2):
        A, B = _large_operands(2100 + i, m, k1, k2, signed)
        _, c_op = xr.gemm_bound(xr.native_operand(A), xr.native_operand(B), m, k2, k1)
        bound_at = lambda t, c_op=c_op: xr.gemm_bound(c_op, xr.native_operand(scaled(t)), m, n, k2)[0]
        tasks.append((A, B, bound_at, _threshold(bound_at, limit, 1 << 61)))
    T = min(tk[3] for tk in tasks)
    p1, p2 = _plan(ctx, signed, m, k2, k1, 20), _plan(ctx, signed, m, n, k2, prefix)
    trip, want_d = [], []
    for i, (A, B, _, _) in enumerate(tasks):
        Am, Bm, Cm = _matrix(ctx, signed, m, k1, 20), _matrix(ctx, signed, k1, k2, 20), _matrix(ctx, signed, m, k2, 20)
        Em, Dm = _matrix(ctx, signed, k2, n, 20), _matrix(ctx, signed, m, n, 20)
        for M, src in ((Am, A), (Bm, B), (Em, scaled(T))):
            assert _pack(ctx, M, src, signed, True) == r.SUCCESS
        r.check(_async_gemm(ctx, p1, Am, Bm, Cm, r.Workspace(ctx, p1)), "C")
        trip.append((Cm, Em, Dm, Am, Bm))
        want_d.append(_int_matmul(_int_matmul(A, B), scaled(T)))
    r.check(r.gemm_rns_grouped(ctx, p2, [(c, e_, d, r.Workspace(ctx, p2)) for c, e_, d, _, _ in trip]), "grouped")
    before = []
    for (_, _, Dm, _, _), (_, _, bound_at, _), w in zip(trip, tasks, want_d):
        assert Dm.exact_proof(ctx)[0] == bound_at(T)
        st, D = _export(ctx, p2, Dm, m, n, signed, prefix)
        assert st == r.SUCCESS and D == w
        before.append((Dm.exact_proof(ctx), Dm.read_residues()))
    for _, Em, _, _, _ in trip:
        assert _pack(ctx, Em, scaled(T + 1), signed, True) == r.SUCCESS
    st = r.gemm_rns_grouped(ctx, p2, [(c, e_, d, r.Workspace(ctx, p2)) for c, e_, d, _, _ in trip])
    assert st == r.RANGE_ERROR
    for (_, _, Dm, _, _), (proof, planes) in zip(trip, before):
        assert Dm.exact_proof(ctx) == proof
        np.testing.assert_array_equal(Dm.read_residues(), planes)
