"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Every comparison is bit-exact: residue planes byte for byte, exports value for
value and status for status, on the same seeded inputs.
"""
import ctypes

import numpy as np
import pytest

import oracle
import rns8_amd as r
from rns8_amd import inputs

pytestmark = pytest.mark.gpu

I64_MIN = np.iinfo(np.int64).min
I64_MAX = np.iinfo(np.int64).max
U64_MAX = np.iinfo(np.uint64).max


def rand_i64(seed, shape, bits=None):
    """Seeded int64 operand; full-range operands also carry the edge values."""
    if bits is not None:
        return inputs.int_range(seed, shape, bits)
    a = inputs.full_int64(seed, shape).copy()
    flat = a.reshape(-1)
    specials = [0, 1, -1, I64_MIN, I64_MAX, I64_MIN + 1, 127, -128, 128, -129]
    flat[: min(len(specials), flat.size)] = specials[: flat.size]
    return a


def rand_u64(seed, shape, bits=None):
    a = inputs.uint_range(seed, shape, bits) if bits else inputs.splitmix64(seed, int(np.prod(shape))).reshape(shape)
    flat = a.reshape(-1)
    specials = np.array([0, 1, U64_MAX, U64_MAX - 1, 255, 256, 1 << 63], dtype=np.uint64)
    flat[: min(len(specials), flat.size)] = specials[: flat.size]
    return a


def bounded_matrix(ctx, rows, cols, semantics, prefix):
    bk = r.BOUND_GLOBAL_MAX_ABS if semantics == r.BOUNDED_I64 else (
        r.BOUND_GLOBAL_MAX_UNSIGNED if semantics == r.BOUNDED_U64 else r.BOUND_NONE)
    return r.Matrix(ctx, r.matrix_desc(rows, cols, semantics, bk, max_prefix=prefix))


@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 5), (33, 17), (255, 259), (64, 4097), (256, 256)])
@pytest.mark.parametrize("prefix", [1, 9, 20])
def test_pack_i64_planes_match_oracle(gpu_ctx, rows, cols, prefix):
    src = rand_i64(rows * 1000 + cols, (rows, cols))
    sem = r.BOUNDED_I64
    m = bounded_matrix(gpu_ctx, rows, cols, sem, prefix)
    r.check(r.pack_i64(gpu_ctx, m, src, 1), "pack")
    got = m.read_residues()
    np.testing.assert_array_equal(got, oracle.pack_i64(src, prefix))


@pytest.mark.parametrize("rows,cols", [(3, 3), (17, 40), (128, 1000)])
def test_pack_u64_planes_match_oracle(gpu_ctx, rows, cols):
    src = rand_u64(rows + 7 * cols, (rows, cols))
    m = bounded_matrix(gpu_ctx, rows, cols, r.BOUNDED_U64, 20)
    r.check(r.pack_u64(gpu_ctx, m, src, 1), "pack")
    np.testing.assert_array_equal(m.read_residues(), oracle.pack_u64(src, 20))


def test_pack_strided_source(gpu_ctx):
    # row stride larger than cols (padded host rows)
    full = rand_i64(5, (20, 37))
    view = full[:, :30]
    m = bounded_matrix(gpu_ctx, 20, 30, r.BOUNDED_I64, 9)
    r.check(r.pack_i64(gpu_ctx, m, full, 1, ld=37), "pack")
    np.testing.assert_array_equal(m.read_residues(), oracle.pack_i64(np.ascontiguousarray(view), 9))


def run_resident_i64(ctx, A, B, prefix, bound, force=True):
    m_, k_ = A.shape
    n_ = B.shape[1]
    flags = r.PLAN_FORCE_FIXED_PREFIX if force else 0
    desc = r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, m_, n_, k_, bound=bound, max_prefix=prefix,
                       flags=flags)
    plan = r.Plan(ctx, desc)
    p = plan.prefix
    Am = bounded_matrix(ctx, m_, k_, r.BOUNDED_I64, p)
    Bm = bounded_matrix(ctx, k_, n_, r.BOUNDED_I64, p)
    Cm = bounded_matrix(ctx, m_, n_, r.BOUNDED_I64, p)
    ws = r.Workspace(ctx, plan)
    r.check(r.pack_i64(ctx, Am, A, 1), "pack A")
    r.check(r.pack_i64(ctx, Bm, B, 2), "pack B")
    r.check(r.gemm_rns(ctx, plan, Am, Bm, Cm, ws), "gemm")
    return plan, Am, Bm, Cm, ws, p


@pytest.mark.parametrize(
    "m,n,k",
    [(1, 1, 1), (2, 3, 4), (7, 9, 13), (64, 64, 64), (256, 256, 256), (300, 200, 150), (257, 513, 129),
     (96, 272, 700)],
)
def test_gemm_planes_match_oracle(gpu_ctx, m, n, k):
    A = rand_i64(m * 31 + k, (m, k), bits=20)
    B = rand_i64(n * 17 + k, (k, n), bits=20)
    bound = k << 40
    plan, Am, Bm, Cm, ws, p = run_resident_i64(gpu_ctx, A, B, 9, bound)
    got = Cm.read_residues(p)
    want = oracle.gemm_rns(oracle.pack_i64(A, p), oracle.pack_i64(B, p), p)
    np.testing.assert_array_equal(got, want)
    out = np.zeros((m, n), dtype=np.int64)
    st = r.export_i64(gpu_ctx, plan, Cm, out)
    ost, oout = oracle.export_i64(want, p, bound)
    assert st == ost == r.SUCCESS
    np.testing.assert_array_equal(out, oout)
    # independent check: brute-force exact integer product (no RNS)
    np.testing.assert_array_equal(out, oracle.exact_gemm_i64(A, B, limbs=1).view(np.int64))


def test_gemm_worst_case_accumulation(gpu_ctx):
    # every product at the int32 extreme (-128 * -128 for m=256) over one safe K block
    k = 65536
    A = np.full((2, k), -128, dtype=np.int64)
    B = np.full((k, 16), -128, dtype=np.int64)
    plan, Am, Bm, Cm, ws, p = run_resident_i64(gpu_ctx, A, B, 9, 1 << 40)
    np.testing.assert_array_equal(Cm.read_residues(p), oracle.gemm_rns(oracle.pack_i64(A, p), oracle.pack_i64(B, p), p))


@pytest.mark.parametrize("k", [65537, 131073])
def test_gemm_k_beyond_safe_block(gpu_ctx, k):
    # reference test_ring_gemm.cpp:46-53 (all-127 K=65537) and multi-block sums
    A = np.full((3, k), 127, dtype=np.int64)
    B = np.full((k, 5), 127, dtype=np.int64)
    A[1, ::3] = -7
    plan, Am, Bm, Cm, ws, p = run_resident_i64(gpu_ctx, A, B, 9, k * 127 * 127)
    np.testing.assert_array_equal(Cm.read_residues(p), oracle.gemm_rns(oracle.pack_i64(A, p), oracle.pack_i64(B, p), p))
    out = np.zeros((3, 5), dtype=np.int64)
    r.check(r.export_i64(gpu_ctx, plan, Cm, out), "export")
    np.testing.assert_array_equal(out, oracle.exact_gemm_i64(A, B, limbs=1).view(np.int64))


def test_export_range_error_preserves_dst(gpu_ctx):
    A = np.array([[1 << 30, 1 << 30]], dtype=np.int64)
    B = np.array([[1 << 30], [1 << 30]], dtype=np.int64)
    # declared bound 10 is false for 2^61
    plan, Am, Bm, Cm, ws, p = run_resident_i64(gpu_ctx, A, B, 9, 10, force=True)
    out = np.full((1, 1), 77, dtype=np.int64)
    assert r.export_i64(gpu_ctx, plan, Cm, out) == r.RANGE_ERROR
    assert out[0, 0] == 77


def test_oneshot_example_known_answer(gpu_ctx):
    # reference examples/bounded_i64_oneshot.cpp:17-27
    desc = r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, 2, 2, 3, bound=100)
    A = np.array([[2, -3, 4], [-5, 6, 7]], dtype=np.int64)
    B = np.array([[1, 8], [-2, 9], [3, -4]], dtype=np.int64)
    st, C = r.gemm_i64_oneshot(gpu_ctx, desc, A, B)
    assert st == r.SUCCESS
    assert C.reshape(-1).tolist() == [20, -27, 4, -14]


def test_config1_oneshot_matches_oracle(gpu_ctx):
    # C1: 256^3, U[-2^20, 2^20), bound K*2^40 -> prefix 7
    A = inputs.int_range(inputs.operand_seed(1, "A"), (256, 256), 20)
    B = inputs.int_range(inputs.operand_seed(1, "B"), (256, 256), 20)
    desc = r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, 256, 256, 256, bound=256 << 40)
    assert r.select_prefix(desc) == (0, 7)
    st, C = r.gemm_i64_oneshot(gpu_ctx, desc, A, B)
    ost, oc = oracle.gemm_i64(A, B, 7, 256 << 40)
    assert st == ost == 0
    np.testing.assert_array_equal(C, oc)


def test_u64_splitk_tall_skinny(gpu_ctx):
    # C5 shape: 128 x 128 x 65536, U[0, 2^23), bound 2^62 -> prefix 8, split-K
    A = inputs.uint_range(inputs.operand_seed(5, "A"), (128, 65536), 23)
    B = inputs.uint_range(inputs.operand_seed(5, "B"), (65536, 128), 23)
    desc = r.gemm_desc(r.BOUNDED_U64, r.BOUND_GLOBAL_MAX_UNSIGNED, 128, 128, 65536, bound=1 << 62)
    st, C = r.gemm_u64_oneshot(gpu_ctx, desc, A, B)
    assert st == 0
    ost, oc = oracle.gemm_u64(A, B, 8, 1 << 62, row0=0, rows=16)
    assert ost == 0
    np.testing.assert_array_equal(C[:16], oc)
    np.testing.assert_array_equal(C[:4, :4], (A[:4].astype(object) @ B[:, :4].astype(object)).astype(np.uint64))


@pytest.mark.parametrize("modulus,field", [(251, True), (2, True), (256, False), (255, False), (7, False)])
def test_finite_oneshot_matches_oracle(gpu_ctx, modulus, field):
    m_, n_, k_ = 130, 70, 300
    A = inputs.bytes_below(11, (m_, k_), 256)
    B = inputs.bytes_below(12, (k_, n_), 256)
    sem = r.FINITE_FIELD_U8 if field else r.FINITE_RING_U8
    desc = r.gemm_desc(sem, r.BOUND_NONE, m_, n_, k_, finite_modulus=modulus)
    st, C = r.gemm_finite_u8_oneshot(gpu_ctx, desc, modulus, A, B, field)
    assert st == 0
    np.testing.assert_array_equal(C, oracle.gemm_finite_u8(A, B, modulus))
    want = ((A.astype(np.int64) @ B.astype(np.int64)) % modulus).astype(np.uint8)
    np.testing.assert_array_equal(C, want)


@pytest.mark.parametrize("prefix,limbs", [(18, 3), (20, 3), (20, 4), (20, 1), (20, 6), (18, 5)])
def test_exact_wide_signed_limbs_match_oracle(gpu_ctx, prefix, limbs):
    m_, n_, k_ = 40, 24, 64
    A = rand_i64(21, (m_, k_))
    B = rand_i64(22, (k_, n_))
    flags = r.PLAN_FORCE_FIXED_PREFIX
    desc = r.gemm_desc(r.EXACT_WIDE_SIGNED, r.BOUND_NONE, m_, n_, k_, max_prefix=prefix, flags=flags)
    plan = r.Plan(gpu_ctx, desc)
    p = plan.prefix
    mk = lambda rows, cols: r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, r.EXACT_WIDE_SIGNED, r.BOUND_NONE, p))
    Am, Bm, Cm = mk(m_, k_), mk(k_, n_), mk(m_, n_)
    ws = r.Workspace(gpu_ctx, plan)
    r.check(r.pack_i64(gpu_ctx, Am, A, 1), "pack A")
    r.check(r.pack_i64(gpu_ctx, Bm, B, 2), "pack B")
    r.check(r.gemm_rns(gpu_ctx, plan, Am, Bm, Cm, ws), "gemm")
    want_planes = oracle.gemm_rns(oracle.pack_i64(A, p), oracle.pack_i64(B, p), p)
    np.testing.assert_array_equal(Cm.read_residues(p), want_planes)
    out = np.full((m_, n_ * limbs), 0xA5A5, dtype=np.uint64)
    st = r.export_exact_wide_signed_limbs(gpu_ctx, plan, Cm, out, limbs)
    ost, oout = oracle.export_exact_wide(want_planes, p, limbs, True)
    assert st == ost
    if st == 0:
        np.testing.assert_array_equal(out, oout)
        exact = oracle.exact_gemm_i64(A, B, limbs=4)
        for i in range(3):
            for j in range(3):
                v = oracle.limbs_to_int(exact[i, 4 * j:4 * j + 4], True)
                assert oracle.limbs_to_int(out[i, limbs * j:limbs * j + limbs], True) == v
    else:
        assert (out == 0xA5A5).all()


@pytest.mark.parametrize("m_,n_", [(45, 530), (3, 257), (300, 1030)])
@pytest.mark.parametrize("signed,prefix,limbs", [(True, 17, 3), (True, 18, 3), (True, 20, 4), (True, 20, 1),
                                                 (True, 19, 5), (False, 18, 3), (False, 20, 2)])
def test_exact_wide_export_multi_chunk_rows(gpu_ctx, m_, n_, signed, prefix, limbs):
    """Exact-wide limb exports whose rows span several 256-cell chunks of the
    matrix-core export (ragged last chunk), with a destination row stride
    above the row length: every limb equals the oracle's export of the same
    planes, RANGE_ERROR leaves the destination untouched."""
    k_ = 24
    sem = r.EXACT_WIDE_SIGNED if signed else r.EXACT_WIDE_UNSIGNED
    A = rand_i64(31 + m_, (m_, k_)) if signed else rand_u64(31 + m_, (m_, k_))
    B = rand_i64(32 + n_, (k_, n_)) if signed else rand_u64(32 + n_, (k_, n_))
    desc = r.gemm_desc(sem, r.BOUND_NONE, m_, n_, k_, max_prefix=prefix, flags=r.PLAN_FORCE_FIXED_PREFIX)
    plan = r.Plan(gpu_ctx, desc)
    assert plan.prefix == prefix
    mk = lambda rows, cols: r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, sem, r.BOUND_NONE, prefix))
    Am, Bm, Cm = mk(m_, k_), mk(k_, n_), mk(m_, n_)
    ws = r.Workspace(gpu_ctx, plan)
    pack = r.pack_i64 if signed else r.pack_u64
    r.check(pack(gpu_ctx, Am, A, 1), "pack A")
    r.check(pack(gpu_ctx, Bm, B, 2), "pack B")
    r.check(r.gemm_rns(gpu_ctx, plan, Am, Bm, Cm, ws), "gemm")
    planes = Cm.read_residues(prefix)
    ld = n_ + 3
    out = np.full((m_, ld * limbs), 0xA5A5, dtype=np.uint64)
    export = r.export_exact_wide_signed_limbs if signed else r.export_exact_wide_unsigned_limbs
    st = export(gpu_ctx, plan, Cm, out, limbs)
    ost, oout = oracle.export_exact_wide(planes, prefix, limbs, signed)
    assert st == ost
    if st == 0:
        np.testing.assert_array_equal(out[:, :n_ * limbs], oout)
        assert (out[:, n_ * limbs:] == 0xA5A5).all()
    else:
        assert (out == 0xA5A5).all()


def test_host_staging_multi_chunk_strided(gpu_ctx):
    """Host operands and results larger than one 16 MB staging chunk, with row
    strides above the row length on both sides (C = A x I round trip)."""
    rows, cols, ld = 2100, 1100, 1111
    full = rand_i64(77, (rows, ld), bits=40)
    n = cols
    B = np.eye(cols, dtype=np.int64)
    desc = r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, rows, n, cols, bound=1 << 40, max_prefix=9,
                       flags=r.PLAN_FORCE_FIXED_PREFIX)
    plan = r.Plan(gpu_ctx, desc)
    Am = bounded_matrix(gpu_ctx, rows, cols, r.BOUNDED_I64, 9)
    Bm = bounded_matrix(gpu_ctx, cols, n, r.BOUNDED_I64, 9)
    Cm = bounded_matrix(gpu_ctx, rows, n, r.BOUNDED_I64, 9)
    ws = r.Workspace(gpu_ctx, plan)
    r.check(r.pack_i64(gpu_ctx, Am, full, 1, ld=ld), "pack A")
    A = np.ascontiguousarray(full[:, :cols])
    np.testing.assert_array_equal(Am.read_residues(9)[:, ::97], oracle.pack_i64(A, 9)[:, ::97])
    r.check(r.pack_i64(gpu_ctx, Bm, B, 2), "pack B")
    r.check(r.gemm_rns(gpu_ctx, plan, Am, Bm, Cm, ws), "gemm")
    out = np.full((rows, n + 7), 5, dtype=np.int64)
    st = r.lib().rns8_export_i64(gpu_ctx.ptr, plan.ptr, Cm.ptr, out.ctypes.data_as(ctypes.c_void_p), n + 7)
    assert st == r.SUCCESS
    np.testing.assert_array_equal(out[:, :n], A)
    assert (out[:, n:] == 5).all()  # padding columns of dst untouched


def test_host_staging_row_longer_than_chunk(gpu_ctx):
    """One row of 17.6 MB: the staging splits inside the row."""
    cols = 2_200_000
    src = rand_i64(78, (1, cols))
    m = bounded_matrix(gpu_ctx, 1, cols, r.BOUNDED_I64, 3)
    r.check(r.pack_i64(gpu_ctx, m, src, 1), "pack")
    np.testing.assert_array_equal(m.read_residues(3), oracle.pack_i64(src, 3))
