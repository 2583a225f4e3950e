"""GPU parity for the fused native-input GEMM's skinny form (results at most
16 columns wide, fused_skinny.hip): C's residue planes from native device
operands must equal, byte for byte, the planes rns8_gemm_rns computes from
packed operands, and export to the exact product.

Cases cover one to 16 columns; 1 to 20 planes (one launch of up to 18
planes, or two launches over the same rows); K below one 64-K
step, K odd, K split into residue slices (above 65536 too); ragged row
blocks; row strides above the width, odd B strides and a B only 8-byte
aligned (B is read by scalar loads); full-range operands; operands that end
exactly at their last logical element; and the 8192 x 1 x 8192 GEMV against
numpy's exact product.
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


def _plan(ctx, signed, m, n, k, prefix, bound):
    sem = r.BOUNDED_I64 if signed else r.BOUNDED_U64
    bk = r.BOUND_GLOBAL_MAX_ABS if signed else r.BOUND_GLOBAL_MAX_UNSIGNED
    plan = r.Plan(ctx, r.gemm_desc(sem, bk, m, n, k, bound=bound, max_prefix=prefix, flags=r.PLAN_FORCE_FIXED_PREFIX))
    assert plan.prefix == prefix
    return plan, sem, bk


def _operands(seed, m, n, k, lda, ldb, signed):
    if signed:
        A = inputs.full_int64(inputs.operand_seed(seed, "A"), (m, lda))
        B = inputs.full_int64(inputs.operand_seed(seed, "B"), (k, ldb))
    else:
        A = inputs.splitmix64(inputs.operand_seed(seed, "A"), m * lda).reshape(m, lda)
        B = inputs.splitmix64(inputs.operand_seed(seed, "B"), k * ldb).reshape(k, ldb)
    return A, B


def _native(ctx, plan, sem, bk, A, B, lda, ldb, signed, b_offset=0):
    """The fused entry on device copies of A and B (B placed b_offset bytes
    into its allocation)."""
    C = r.Matrix(ctx, r.matrix_desc(plan.desc.m, plan.desc.n, sem, bk, plan.prefix))
    ws = r.Workspace(ctx, plan)
    dA = hip.malloc(A.nbytes)
    dB = hip.malloc(B.nbytes + 16)
    try:
        hip.to_device(dA, np.ascontiguousarray(A))
        hip.to_device(dB + b_offset, np.ascontiguousarray(B))
        fn = r.lib().rns8_mi355x_gemm_native_i64_async if signed else r.lib().rns8_mi355x_gemm_native_u64_async
        st = fn(ctx.ptr, plan.ptr, _vp(dA), lda, _vp(dB + b_offset), ldb, C.ptr, ws.ptr, None)
        hip.synchronize()
    finally:
        hip.free(dA)
        hip.free(dB)
    return st, C


def _packed(ctx, plan, sem, bk, A, B, lda, ldb, signed):
    m, n, k, p = plan.desc.m, plan.desc.n, plan.desc.k, plan.prefix
    Am = r.Matrix(ctx, r.matrix_desc(m, k, sem, bk, p))
    Bm = r.Matrix(ctx, r.matrix_desc(k, n, sem, bk, p))
    Cm = r.Matrix(ctx, r.matrix_desc(m, n, sem, bk, p))
    pack = r.pack_i64 if signed else r.pack_u64
    r.check(pack(ctx, Am, A, 1, ld=lda), "pack A")
    r.check(pack(ctx, Bm, B, 2, ld=ldb), "pack B")
    r.check(r.gemm_rns(ctx, plan, Am, Bm, Cm, r.Workspace(ctx, plan)), "gemm")
    return Cm


# (m, n, k, prefix, lda_extra, ldb_extra, signed, b_offset); A's stride is even
CASES = [
    (1000, 1, 8192, 9, 0, 0, True, 0),       # GEMV, one launch of nine planes, K split
    (1000, 3, 3001, 9, 3, 1, True, 8),       # odd K, strides above the width, B 8-byte aligned
    (33, 16, 70001, 5, 1, 0, False, 0),      # 16 columns, K above 65536
    (16, 8, 200000, 9, 0, 5, True, 0),       # one row block, many slices
    (7, 2, 40, 3, 2, 0, False, 0),           # K below one step, rows below one block
    (100, 5, 999, 20, 3, 0, True, 0),        # 20 planes: two launches of 10
    (50, 16, 5000, 10, 0, 0, False, 0),      # 10 planes in one launch
    (200, 2, 3000, 18, 0, 0, True, 0),       # 18 planes in one launch (the largest group)
    (300, 4, 1, 1, 1, 3, True, 8),           # K = 1, one plane (m = 256)
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_fused_skinny_planes_equal_packed_gemm(gpu_ctx, case):
    m, n, k, prefix, lda_x, ldb_x, signed, b_off = CASES[case]
    lda, ldb = k + lda_x, n + ldb_x
    assert lda % 2 == 0
    A, B = _operands(1300 + case, m, n, k, lda, ldb, signed)
    plan, sem, bk = _plan(gpu_ctx, signed, m, n, k, prefix, 2)
    st, C = _native(gpu_ctx, plan, sem, bk, A, B, lda, ldb, signed, b_off)
    assert st == r.SUCCESS
    Cp = _packed(gpu_ctx, plan, sem, bk, A, B, lda, ldb, signed)
    np.testing.assert_array_equal(C.read_residues(), Cp.read_residues())
    if m * n * k <= 1 << 22:
        opack = oracle.pack_i64 if signed else oracle.pack_u64
        want = oracle.gemm_rns(opack(np.ascontiguousarray(A[:, :k]), prefix),
                               opack(np.ascontiguousarray(B[:, :n]), prefix), prefix)
        np.testing.assert_array_equal(C.read_residues(), want)


@pytest.mark.parametrize("signed", [True, False])
def test_fused_skinny_reads_stay_in_logical_extent(gpu_ctx, signed):
    """A in a buffer of exactly (m - 1) * lda + k elements and B of (k - 1) *
    ldb + n, each at the very end of a 64 KiB-aligned allocation: no load
    reaches past the last logical element, and the planes equal the packed
    GEMM's."""
    m, n, k, prefix = 70, 3, 3002, 9  # A's start stays 16-byte aligned: (m - 1) * lda + k is even
    lda, ldb = k + 30, n + 5
    A, B = _operands(1400 + signed, m, n, k, lda, ldb, signed)
    plan, sem, bk = _plan(gpu_ctx, signed, m, n, k, prefix, 2)
    a_elems, b_elems = (m - 1) * lda + k, (k - 1) * ldb + n
    a_alloc = (a_elems * 8 + 65535) // 65536 * 65536
    b_alloc = (b_elems * 8 + 65535) // 65536 * 65536
    C = r.Matrix(gpu_ctx, r.matrix_desc(m, n, sem, bk, prefix))
    ws = r.Workspace(gpu_ctx, plan)
    baseA, baseB = hip.malloc(a_alloc), hip.malloc(b_alloc)
    try:
        dA, dB = baseA + a_alloc - a_elems * 8, baseB + b_alloc - b_elems * 8
        assert dA % 16 == 0
        hip.to_device(dA, np.ascontiguousarray(A.reshape(-1)[:a_elems]))
        hip.to_device(dB, np.ascontiguousarray(B.reshape(-1)[:b_elems]))
        fn = r.lib().rns8_mi355x_gemm_native_i64_async if signed else r.lib().rns8_mi355x_gemm_native_u64_async
        st = fn(gpu_ctx.ptr, plan.ptr, _vp(dA), lda, _vp(dB), ldb, C.ptr, ws.ptr, None)
        hip.synchronize()
    finally:
        hip.free(baseA)
        hip.free(baseB)
    assert st == r.SUCCESS
    Cp = _packed(gpu_ctx, plan, sem, bk, A, B, lda, ldb, signed)
    np.testing.assert_array_equal(C.read_residues(), Cp.read_residues())


def test_fused_skinny_refuses_unaligned_a(gpu_ctx):
    m, n, k = 64, 1, 1024
    plan, sem, bk = _plan(gpu_ctx, True, m, n, k, 9, 1 << 62)
    C = r.Matrix(gpu_ctx, r.matrix_desc(m, n, sem, bk, 9))
    ws = r.Workspace(gpu_ctx, plan)
    dA, dB = hip.malloc(m * (k + 1) * 8 + 64), hip.malloc(k * 8 + 64)
    try:
        fn = r.lib().rns8_mi355x_gemm_native_i64_async
        # odd A stride, then A only 8-byte aligned: refused before any kernel runs
        assert fn(gpu_ctx.ptr, plan.ptr, _vp(dA), k + 1, _vp(dB), n, C.ptr, ws.ptr, None) == r.UNSUPPORTED_BACKEND
        assert fn(gpu_ctx.ptr, plan.ptr, _vp(dA + 8), k, _vp(dB), n, C.ptr, ws.ptr, None) == r.UNSUPPORTED_BACKEND
        hip.synchronize()
    finally:
        hip.free(dA)
        hip.free(dB)


@pytest.mark.parametrize("signed", [True, False])
def test_fused_gemv_full_size_export(gpu_ctx, signed):
    # the bench's 8192 x 1 x 8192 at prefix 9; |sum| < 8192 * 2^40 = 2^53, so
    # numpy's int64 product is exact
    m, k = 8192, 8192
    if signed:
        A = inputs.int_range(1501, (m, k), 20)
        B = inputs.int_range(1502, (k, 1), 20)
    else:
        A = inputs.uint_range(1501, (m, k), 20)
        B = inputs.uint_range(1502, (k, 1), 20)
    plan, sem, bk = _plan(gpu_ctx, signed, m, 1, k, 9, k << 40)
    st, C = _native(gpu_ctx, plan, sem, bk, A, B, k, 1, signed)
    assert st == r.SUCCESS
    out = np.zeros((m, 1), dtype=np.int64 if signed else np.uint64)
    r.check((r.export_i64 if signed else r.export_u64)(gpu_ctx, plan, C, out), "export")
    want = A.astype(np.int64) @ B.astype(np.int64)
    np.testing.assert_array_equal(out.astype(np.int64), want)
