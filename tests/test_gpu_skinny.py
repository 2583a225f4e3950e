"""GPU parity for narrow results and K splits.

Results at most 16 columns wide run the skinny kernel (16 rows per MFMA
block, A streamed straight into registers, K split into int8 residue slices
when rows x planes are few); wider results with few output tiles split the
whole K of one plane_gemm_kernel launch into int8 residue slices. Every case
compares the residue planes byte for byte with the oracle and the exported
values with a brute-force integer product (reference shapes: the N <= 8 GEMV
of hip_direct_gemm_tiled_kernels.cuh:298-432 and the M*N <= 64 kernel of
hip_direct_gemm_kernels.cuh:10-35).
"""
import numpy as np
import pytest

import oracle
import rns8_amd as r
from rns8_amd import inputs

pytestmark = pytest.mark.gpu


def _run_i64(ctx, A, B, prefix, bound):
    m, k = A.shape
    n = B.shape[1]
    desc = r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, m, n, k, bound=bound, max_prefix=prefix,
                       flags=r.PLAN_FORCE_FIXED_PREFIX)
    plan = r.Plan(ctx, desc)
    p = plan.prefix
    mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, p))
    Am, Bm, Cm = mk(m, k), mk(k, n), mk(m, n)
    ws = r.Workspace(ctx, plan)
    r.check(r.pack_i64(ctx, Am, A, 1), "pack A")
    r.check(r.pack_i64(ctx, Bm, B, 2), "pack B")
    r.check(r.gemm_rns(ctx, plan, Am, Bm, Cm, ws), "gemm")
    return plan, Cm, p


def _check(ctx, A, B, prefix, bound):
    plan, Cm, p = _run_i64(ctx, A, B, prefix, bound)
    want = oracle.gemm_rns(oracle.pack_i64(A, p), oracle.pack_i64(B, p), p)
    np.testing.assert_array_equal(Cm.read_residues(p), want)
    out = np.zeros((A.shape[0], B.shape[1]), dtype=np.int64)
    r.check(r.export_i64(ctx, plan, Cm, out), "export")
    np.testing.assert_array_equal(out, oracle.exact_gemm_i64(A, B, limbs=1).view(np.int64))
    return plan


@pytest.mark.parametrize(
    "m,n,k",
    [
        (1000, 1, 3000),    # GEMV, 2 row blocks per wave, ragged last row group and K step
        (4097, 8, 2048),    # N = 8, one row past a row group
        (33, 16, 5000),     # 2 row blocks per wave, one row in the second group
        (16, 5, 20000),     # 1 row block per wave, K split
        (8, 8, 300000),     # M*N = 64, K beyond 65536: several int32-safe slices
        (1, 1, 70001),      # single cell, ragged K
        (3000, 16, 127),    # K shorter than one pipeline step
    ],
)
def test_skinny_matches_oracle(gpu_ctx, m, n, k):
    A = inputs.int_range(m * 131 + k, (m, k), 20)
    B = inputs.int_range(n * 71 + k, (k, n), 20)
    plan = _check(gpu_ctx, A, B, 9, k << 40)
    assert plan.selected_kernel().startswith("skinny_gemm_kernel")


def test_skinny_full_range_planes(gpu_ctx):
    # full-range int64 operands at prefix 20 (every ladder modulus, m = 256
    # among them), residues only: the product exceeds int64
    m, n, k = 300, 4, 3000
    A = inputs.full_int64(5101, (m, k))
    B = inputs.full_int64(5102, (k, n))
    plan, Cm, p = _run_i64(gpu_ctx, A, B, 20, 1 << 62)
    assert p == 20
    np.testing.assert_array_equal(Cm.read_residues(p), oracle.gemm_rns(oracle.pack_i64(A, p), oracle.pack_i64(B, p), p))


def test_skinny_u64_oneshot(gpu_ctx):
    m, n, k = 513, 3, 9000
    A = inputs.uint_range(7001, (m, k), 23)
    B = inputs.uint_range(7002, (k, n), 23)
    desc = r.gemm_desc(r.BOUNDED_U64, r.BOUND_GLOBAL_MAX_UNSIGNED, m, n, k, bound=1 << 62)
    st, C = r.gemm_u64_oneshot(gpu_ctx, desc, A, B)
    assert st == r.SUCCESS
    np.testing.assert_array_equal(C, (A.astype(object) @ B.astype(object)).astype(np.uint64))


@pytest.mark.parametrize("m,n,k", [(64, 40, 140000), (100, 130, 9000)])
def test_wide_k_split_matches_oracle(gpu_ctx, m, n, k):
    # plane_gemm_kernel with one launch over the whole K in int8 residue slices
    A = inputs.int_range(m * 7 + k, (m, k), 18)
    B = inputs.int_range(n * 5 + k, (k, n), 18)
    plan = _check(gpu_ctx, A, B, 9, k << 36)
    assert "K split" in plan.selected_kernel()


@pytest.mark.parametrize("modulus,field", [(251, True), (256, False), (2, True), (255, False)])
def test_skinny_finite_oneshot(gpu_ctx, modulus, field):
    # one finite plane on the skinny kernel, K split into residue slices
    m, n, k = 300, 7, 20000
    A = inputs.bytes_below(modulus + 1, (m, k), 256)
    B = inputs.bytes_below(modulus + 2, (k, n), 256)
    sem = r.FINITE_FIELD_U8 if field else r.FINITE_RING_U8
    desc = r.gemm_desc(sem, r.BOUND_NONE, m, n, k, finite_modulus=modulus)
    st, C = r.gemm_finite_u8_oneshot(gpu_ctx, desc, modulus, A, B, field)
    assert st == 0
    np.testing.assert_array_equal(C, oracle.gemm_finite_u8(A, B, modulus))
    np.testing.assert_array_equal(C, ((A.astype(np.int64) @ B.astype(np.int64)) % modulus).astype(np.uint8))
