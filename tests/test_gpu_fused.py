"""Fused native-input GEMM (rns8_mi355x_gemm_native_i64/u64_async): C's
residue planes straight from native device operands must equal, byte for
byte, the planes rns8_gemm_rns computes from packed operands (and the oracle's
for small cases), and export to the exact product.

Cases cover: one and several 128 x 128 output tiles with ragged edges; plane
counts 1, 3, 4, 5, 8, 9 and 20 (full groups of four planes and tails of one to
three); K below one step, K not a multiple of 32, K above 65536 (several
slices); row strides above the width; full-range int64/uint64 operands (every
byte of the inputs matters for the residues); and the refusals: the 4096 x
4096 plan the fused path is not offered for, odd row strides and operands not
16-byte aligned (its loads move 16-byte chunks straight into LDS).
"""
import ctypes

import numpy as np
import pytest

import oracle
import rns8_amd as r
from rns8_amd import hip, inputs

pytestmark = pytest.mark.gpu


def _vp(x):
    return ctypes.c_void_p(x)


def _device(arr):
    d = hip.malloc(max(arr.nbytes, 16))
    hip.to_device(d, np.ascontiguousarray(arr))
    return d


def _plans(ctx, signed, m, n, k, prefix, bound):
    sem = r.BOUNDED_I64 if signed else r.BOUNDED_U64
    bk = r.BOUND_GLOBAL_MAX_ABS if signed else r.BOUND_GLOBAL_MAX_UNSIGNED
    plan = r.Plan(ctx, r.gemm_desc(sem, bk, m, n, k, bound=bound, max_prefix=prefix, flags=r.PLAN_FORCE_FIXED_PREFIX))
    return plan, sem, bk


def _fused(ctx, plan, sem, bk, A, B, m, n, k, prefix, lda, ldb, signed):
    """Runs the fused entry on device copies of A (m x lda) and B (k x ldb)."""
    C = r.Matrix(ctx, r.matrix_desc(m, n, sem, bk, prefix))
    ws = r.Workspace(ctx, plan)
    dA, dB = _device(A), _device(B)
    try:
        fn = r.lib().rns8_mi355x_gemm_native_i64_async if signed else r.lib().rns8_mi355x_gemm_native_u64_async
        st = fn(ctx.ptr, plan.ptr, _vp(dA), lda, _vp(dB), ldb, C.ptr, ws.ptr, None)
        hip.synchronize()
    finally:
        hip.free(dA)
        hip.free(dB)
    return st, C


def _packed(ctx, plan, sem, bk, A, B, m, n, k, prefix, lda, ldb, signed):
    Am = r.Matrix(ctx, r.matrix_desc(m, k, sem, bk, prefix))
    Bm = r.Matrix(ctx, r.matrix_desc(k, n, sem, bk, prefix))
    Cm = r.Matrix(ctx, r.matrix_desc(m, n, sem, bk, prefix))
    pack = r.pack_i64 if signed else r.pack_u64
    r.check(pack(ctx, Am, A, 1, ld=lda), "pack A")
    r.check(pack(ctx, Bm, B, 2, ld=ldb), "pack B")
    r.check(r.gemm_rns(ctx, plan, Am, Bm, Cm, r.Workspace(ctx, plan)), "gemm")
    return Cm


def _operands(seed, m, n, k, lda, ldb, signed):
    if signed:
        A = inputs.full_int64(inputs.operand_seed(seed, "A"), (m, lda))
        B = inputs.full_int64(inputs.operand_seed(seed, "B"), (k, ldb))
    else:
        A = inputs.splitmix64(inputs.operand_seed(seed, "A"), m * lda).reshape(m, lda)
        B = inputs.splitmix64(inputs.operand_seed(seed, "B"), k * ldb).reshape(k, ldb)
    return A, B


# (m, n, k, prefix, lda_extra, ldb_extra, signed)
PLANE_CASES = [
    (128, 128, 65536, 8, 0, 0, False),   # the C5 shape
    (100, 70, 3000, 9, 0, 0, True),      # ragged single tile, 4 + 4 + 1 planes
    (1, 1, 1, 1, 1, 1, True),            # one element, one plane (strides padded to even)
    (1, 1, 31, 3, 1, 1, False),          # K below one step
    (130, 257, 5000, 5, 6, 3, True),     # 2 x 3 tiles, 4 + 1 planes, strided
    (64, 64, 70000, 7, 0, 0, False),     # K above 65536: several slices, 4 + 3 planes
    (256, 128, 1000, 20, 0, 0, True),    # five full plane groups
    (77, 45, 999, 4, 1, 3, True),        # ragged everything, strides above the width
    (33, 129, 4097, 2, 1, 1, False),     # two planes, a second tile column of one
]


@pytest.mark.parametrize("case", range(len(PLANE_CASES)))
def test_fused_planes_equal_packed_gemm(gpu_ctx, case):
    m, n, k, prefix, xa, xb, signed = PLANE_CASES[case]
    lda, ldb = k + xa, n + xb
    A, B = _operands(900 + case, m, n, k, lda, ldb, signed)
    # full-range operands: the planes are the product's residues whatever the
    # declared bound, which only matters to the export
    plan, sem, bk = _plans(gpu_ctx, signed, m, n, k, prefix, 1 if prefix == 1 else 2)
    st, Cf = _fused(gpu_ctx, plan, sem, bk, A, B, m, n, k, prefix, lda, ldb, signed)
    assert st == r.SUCCESS
    Cp = _packed(gpu_ctx, plan, sem, bk, A, B, m, n, k, prefix, lda, ldb, signed)
    np.testing.assert_array_equal(Cf.read_residues(), Cp.read_residues())
    if m * n * k <= 1 << 24:
        opack = oracle.pack_i64 if signed else oracle.pack_u64
        Ap = opack(np.ascontiguousarray(A[:, :k]), prefix)
        Bp = opack(np.ascontiguousarray(B[:, :n]), prefix)
        np.testing.assert_array_equal(Cf.read_residues(), oracle.gemm_rns(Ap, Bp, prefix))


@pytest.mark.parametrize("signed", [True, False])
def test_fused_export_is_exact(gpu_ctx, signed):
    m, n, k, prefix = 128, 96, 20000, 9
    if signed:
        A = inputs.int_range(inputs.operand_seed(950, "A"), (m, k), 20)
        B = inputs.int_range(inputs.operand_seed(950, "B"), (k, n), 20)
    else:
        A = (inputs.splitmix64(inputs.operand_seed(951, "A"), m * k) >> np.uint64(44)).reshape(m, k)
        B = (inputs.splitmix64(inputs.operand_seed(951, "B"), k * n) >> np.uint64(44)).reshape(k, n)
    plan, sem, bk = _plans(gpu_ctx, signed, m, n, k, prefix, 1 << 60)
    st, Cf = _fused(gpu_ctx, plan, sem, bk, A, B, m, n, k, prefix, k, n, signed)
    assert st == r.SUCCESS
    out = np.zeros((m, n), dtype=np.int64 if signed else np.uint64)
    export = r.export_i64 if signed else r.export_u64
    r.check(export(gpu_ctx, plan, Cf, out), "export")
    # one 64-bit limb holds every product here (|C| < 2^55)
    want = oracle.exact_gemm_i64(A, B, limbs=1) if signed else oracle.exact_gemm_u64(A, B, limbs=1)
    np.testing.assert_array_equal(out, want.view(out.dtype))


def test_fused_not_offered_for_large_outputs(gpu_ctx):
    m = n = k = 4096
    plan, sem, bk = _plans(gpu_ctx, True, m, n, k, 9, 1 << 62)
    C = r.Matrix(gpu_ctx, r.matrix_desc(m, n, sem, bk, 9))
    ws = r.Workspace(gpu_ctx, plan)
    L = r.lib()
    st = L.rns8_mi355x_gemm_native_i64_async(gpu_ctx.ptr, plan.ptr, _vp(16), k, _vp(16), n, C.ptr, ws.ptr, None)
    assert st == r.UNSUPPORTED_BACKEND


def test_fused_rejects_mismatched_arguments(gpu_ctx):
    m, n, k = 64, 64, 1024
    plan, sem, bk = _plans(gpu_ctx, True, m, n, k, 9, 1 << 62)
    C = r.Matrix(gpu_ctx, r.matrix_desc(m, n, sem, bk, 9))
    wrong = r.Matrix(gpu_ctx, r.matrix_desc(m, n + 1, sem, bk, 9))
    ws = r.Workspace(gpu_ctx, plan)
    L = r.lib()
    # no kernel runs for any of these: the checks come first
    assert L.rns8_mi355x_gemm_native_i64_async(gpu_ctx.ptr, plan.ptr, None, k, _vp(16), n, C.ptr, ws.ptr,
                                               None) == r.INVALID_ARGUMENT
    assert L.rns8_mi355x_gemm_native_i64_async(gpu_ctx.ptr, plan.ptr, _vp(16), k - 1, _vp(16), n, C.ptr, ws.ptr,
                                               None) == r.INVALID_ARGUMENT
    assert L.rns8_mi355x_gemm_native_i64_async(gpu_ctx.ptr, plan.ptr, _vp(16), k, _vp(16), n, wrong.ptr, ws.ptr,
                                               None) == r.INVALID_ARGUMENT
    # the unsigned entry on a signed plan
    assert L.rns8_mi355x_gemm_native_u64_async(gpu_ctx.ptr, plan.ptr, _vp(16), k, _vp(16), n, C.ptr, ws.ptr,
                                               None) == r.INVALID_ARGUMENT


@pytest.mark.parametrize("lda_extra,ldb_extra,offset", [(1, 0, 0), (0, 1, 0), (0, 0, 8)])
def test_fused_refuses_unaligned_operands(gpu_ctx, lda_extra, ldb_extra, offset):
    m, n, k = 64, 64, 1024  # even widths: each extra element makes a stride odd
    lda, ldb = k + lda_extra, n + ldb_extra
    plan, sem, bk = _plans(gpu_ctx, True, m, n, k, 9, 1 << 62)
    C = r.Matrix(gpu_ctx, r.matrix_desc(m, n, sem, bk, 9))
    ws = r.Workspace(gpu_ctx, plan)
    dA, dB = hip.malloc(m * lda * 8 + 64), hip.malloc(k * ldb * 8 + 64)
    try:
        # refused before any kernel runs
        st = r.lib().rns8_mi355x_gemm_native_i64_async(gpu_ctx.ptr, plan.ptr, _vp(dA + offset), lda, _vp(dB), ldb,
                                                       C.ptr, ws.ptr, None)
        hip.synchronize()
    finally:
        hip.free(dA)
        hip.free(dB)
    assert st == r.UNSUPPORTED_BACKEND


@pytest.mark.parametrize("signed", [True, False])
def test_fused_reads_stay_in_logical_extent(gpu_ctx, signed):
    """Strided operands in buffers of exactly (m - 1) * lda + k and
    (k - 1) * ldb + n elements, each placed at the very end of a 64 KiB-aligned
    allocation: the loads' ranges end at the last logical element, so the
    padding of the last row, which such a buffer does not hold, is never
    read, and the planes equal the packed GEMM's."""
    m, n, k, prefix = 130, 200, 3000, 9
    lda, ldb = k + 30, n + 126  # the padding the loads of the last row would cover
    A, B = _operands(970 + signed, m, n, k, lda, ldb, signed)
    plan, sem, bk = _plans(gpu_ctx, signed, m, n, k, prefix, 2)
    a_elems, b_elems = (m - 1) * lda + k, (k - 1) * ldb + n
    a_bytes, b_bytes = a_elems * 8, b_elems * 8
    a_alloc = (a_bytes + 65535) // 65536 * 65536
    b_alloc = (b_bytes + 65535) // 65536 * 65536
    C = r.Matrix(gpu_ctx, r.matrix_desc(m, n, sem, bk, prefix))
    ws = r.Workspace(gpu_ctx, plan)
    baseA, baseB = hip.malloc(a_alloc), hip.malloc(b_alloc)
    try:
        dA, dB = baseA + a_alloc - a_bytes, baseB + b_alloc - b_bytes
        assert dA % 16 == 0 and dB % 16 == 0
        hip.to_device(dA, np.ascontiguousarray(A.reshape(-1)[:a_elems]))
        hip.to_device(dB, np.ascontiguousarray(B.reshape(-1)[:b_elems]))
        fn = r.lib().rns8_mi355x_gemm_native_i64_async if signed else r.lib().rns8_mi355x_gemm_native_u64_async
        st = fn(gpu_ctx.ptr, plan.ptr, _vp(dA), lda, _vp(dB), ldb, C.ptr, ws.ptr, None)
        hip.synchronize()
    finally:
        hip.free(baseA)
        hip.free(baseB)
    assert st == r.SUCCESS
    Cp = _packed(gpu_ctx, plan, sem, bk, A, B, m, n, k, prefix, lda, ldb, signed)
    np.testing.assert_array_equal(C.read_residues(), Cp.read_residues())


def test_fused_refusal_leaves_result_current(gpu_ctx):
    """A refused call (odd stride) enqueues nothing and leaves C as it was: a
    result computed before it still exports."""
    m, n, k, prefix = 64, 64, 1024, 9
    A = inputs.int_range(inputs.operand_seed(980, "A"), (m, k), 20)
    B = inputs.int_range(inputs.operand_seed(980, "B"), (k, n), 20)
    plan, sem, bk = _plans(gpu_ctx, True, m, n, k, prefix, 1 << 60)
    C = r.Matrix(gpu_ctx, r.matrix_desc(m, n, sem, bk, prefix))
    ws = r.Workspace(gpu_ctx, plan)
    dA, dB = _device(A), _device(B)
    try:
        fn = r.lib().rns8_mi355x_gemm_native_i64_async
        assert fn(gpu_ctx.ptr, plan.ptr, _vp(dA), k, _vp(dB), n, C.ptr, ws.ptr, None) == r.SUCCESS
        hip.synchronize()
        assert fn(gpu_ctx.ptr, plan.ptr, _vp(dA), k - 1, _vp(dB), n, C.ptr, ws.ptr, None) == r.INVALID_ARGUMENT
        assert fn(gpu_ctx.ptr, plan.ptr, _vp(dA + 8), k, _vp(dB), n, C.ptr, ws.ptr, None) == r.UNSUPPORTED_BACKEND
        hip.synchronize()
    finally:
        hip.free(dA)
        hip.free(dB)
    out = np.zeros((m, n), dtype=np.int64)
    r.check(r.export_i64(gpu_ctx, plan, C, out), "export after refused calls")
    np.testing.assert_array_equal(out, oracle.exact_gemm_i64(A, B, limbs=1).view(np.int64))
