"""Resident GEMM chains: the result matrix of one rns8_gemm_rns is an operand of
the next, without leaving HBM (reference api_gemm.cpp:838-983 with
exact_range.hpp:104-171 carrying the output's magnitude proof).

* exact-wide signed: D = (A x B) x E is exported exactly, and a chain whose
  carried proof exceeds the prefix's range is refused with RANGE_ERROR;
* bounded int64: the second product is exported exactly under its declared
  bound.
"""
import numpy as np
import pytest

import oracle
import rns8_amd as r
from rns8_amd import inputs

pytestmark = pytest.mark.gpu


def _mk(ctx, rows, cols, sem, bk, prefix):
    return r.Matrix(ctx, r.matrix_desc(rows, cols, sem, bk, prefix))


def test_exact_wide_chain(gpu_ctx):
    m, k1, k2, n = 40, 30, 20, 36
    sem, bk = r.EXACT_WIDE_SIGNED, r.BOUND_NONE
    A = inputs.int_range(inputs.operand_seed(61, "A"), (m, k1), 40)
    B = inputs.int_range(inputs.operand_seed(61, "B"), (k1, k2), 40)
    E = inputs.int_range(inputs.operand_seed(61 + 1000, "B"), (k2, n), 40)
    p1 = r.Plan(gpu_ctx, r.gemm_desc(sem, bk, m, k2, k1, max_prefix=20, flags=r.PLAN_FORCE_FIXED_PREFIX))
    p2 = r.Plan(gpu_ctx, r.gemm_desc(sem, bk, m, n, k2, max_prefix=20, flags=r.PLAN_FORCE_FIXED_PREFIX))
    Am, Bm, Cm = _mk(gpu_ctx, m, k1, sem, bk, 20), _mk(gpu_ctx, k1, k2, sem, bk, 20), _mk(gpu_ctx, m, k2, sem, bk, 20)
    Em, Dm = _mk(gpu_ctx, k2, n, sem, bk, 20), _mk(gpu_ctx, m, n, sem, bk, 20)
    r.check(r.pack_i64(gpu_ctx, Am, A, 1), "pack A")
    r.check(r.pack_i64(gpu_ctx, Bm, B, 2), "pack B")
    r.check(r.pack_i64(gpu_ctx, Em, E, 3), "pack E")
    r.check(r.gemm_rns(gpu_ctx, p1, Am, Bm, Cm, r.Workspace(gpu_ctx, p1)), "C = A x B")
    r.check(r.gemm_rns(gpu_ctx, p2, Cm, Em, Dm, r.Workspace(gpu_ctx, p2)), "D = C x E")
    limbs = 3
    out = np.zeros((m, n * limbs), dtype=np.uint64)
    r.check(r.export_exact_wide_signed_limbs(gpu_ctx, p2, Dm, out, limbs), "export D")
    want = (A.astype(object) @ B.astype(object)) @ E.astype(object)
    for i in range(m):
        for j in range(n):
            assert oracle.limbs_to_int(out[i, limbs * j:limbs * j + limbs], True) == want[i, j], (i, j)


def test_exact_wide_chain_beyond_range_is_refused(gpu_ctx):
    # |C| may reach k1 * 2^126, so C x E can exceed the prefix-20 range (~2^154.8)
    m, k1, k2, n = 8, 16, 16, 8
    sem, bk = r.EXACT_WIDE_SIGNED, r.BOUND_NONE
    A = inputs.full_int64(inputs.operand_seed(62, "A"), (m, k1))
    B = inputs.full_int64(inputs.operand_seed(62, "B"), (k1, k2))
    E = inputs.full_int64(inputs.operand_seed(62 + 1000, "B"), (k2, n))
    p1 = r.Plan(gpu_ctx, r.gemm_desc(sem, bk, m, k2, k1, max_prefix=20, flags=r.PLAN_FORCE_FIXED_PREFIX))
    p2 = r.Plan(gpu_ctx, r.gemm_desc(sem, bk, m, n, k2, max_prefix=20, flags=r.PLAN_FORCE_FIXED_PREFIX))
    Am, Bm, Cm = _mk(gpu_ctx, m, k1, sem, bk, 20), _mk(gpu_ctx, k1, k2, sem, bk, 20), _mk(gpu_ctx, m, k2, sem, bk, 20)
    Em, Dm = _mk(gpu_ctx, k2, n, sem, bk, 20), _mk(gpu_ctx, m, n, sem, bk, 20)
    r.check(r.pack_i64(gpu_ctx, Am, A, 1), "pack A")
    r.check(r.pack_i64(gpu_ctx, Bm, B, 2), "pack B")
    r.check(r.pack_i64(gpu_ctx, Em, E, 3), "pack E")
    r.check(r.gemm_rns(gpu_ctx, p1, Am, Bm, Cm, r.Workspace(gpu_ctx, p1)), "C = A x B")
    assert r.gemm_rns(gpu_ctx, p2, Cm, Em, Dm, r.Workspace(gpu_ctx, p2)) == r.RANGE_ERROR


def test_bounded_chain(gpu_ctx):
    m, k1, k2, n = 50, 40, 30, 60
    sem, bk = r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS
    A = inputs.int_range(inputs.operand_seed(63, "A"), (m, k1), 12)
    B = inputs.int_range(inputs.operand_seed(63, "B"), (k1, k2), 12)
    E = inputs.int_range(inputs.operand_seed(63 + 1000, "B"), (k2, n), 12)
    bound = 1 << 50  # |D| <= 30 * 40 * 2^36 < 2^47
    desc1 = r.gemm_desc(sem, bk, m, k2, k1, bound=bound, max_prefix=9, flags=r.PLAN_FORCE_FIXED_PREFIX)
    desc2 = r.gemm_desc(sem, bk, m, n, k2, bound=bound, max_prefix=9, flags=r.PLAN_FORCE_FIXED_PREFIX)
    p1, p2 = r.Plan(gpu_ctx, desc1), r.Plan(gpu_ctx, desc2)
    Am, Bm, Cm = _mk(gpu_ctx, m, k1, sem, bk, 9), _mk(gpu_ctx, k1, k2, sem, bk, 9), _mk(gpu_ctx, m, k2, sem, bk, 9)
    Em, Dm = _mk(gpu_ctx, k2, n, sem, bk, 9), _mk(gpu_ctx, m, n, sem, bk, 9)
    r.check(r.pack_i64(gpu_ctx, Am, A, 1), "pack A")
    r.check(r.pack_i64(gpu_ctx, Bm, B, 2), "pack B")
    r.check(r.pack_i64(gpu_ctx, Em, E, 3), "pack E")
    r.check(r.gemm_rns(gpu_ctx, p1, Am, Bm, Cm, r.Workspace(gpu_ctx, p1)), "C = A x B")
    r.check(r.gemm_rns(gpu_ctx, p2, Cm, Em, Dm, r.Workspace(gpu_ctx, p2)), "D = C x E")
    out = np.zeros((m, n), dtype=np.int64)
    r.check(r.export_i64(gpu_ctx, p2, Dm, out), "export D")
    np.testing.assert_array_equal(out, (A @ B) @ E)
