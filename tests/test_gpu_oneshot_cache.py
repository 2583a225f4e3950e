"""Repeated oneshot calls on one context reuse the previous call's device
state when the descriptor is equal; every call must still see its own inputs.
Alternating data and descriptors checks that nothing stale is exported."""
import numpy as np
import pytest

import oracle
import rns8_amd as r
from rns8_amd import inputs

pytestmark = pytest.mark.gpu


def test_bounded_oneshot_repeats_see_new_inputs(gpu_ctx):
    m, n, k = 130, 70, 90
    d1 = r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, m, n, k, bound=1 << 50)
    d2 = r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, m, n, k + 1, bound=1 << 50)
    for step, desc in enumerate([d1, d1, d2, d1, d1]):
        kk = desc.k
        A = inputs.int_range(inputs.operand_seed(300 + step, "A"), (m, kk), 20)
        B = inputs.int_range(inputs.operand_seed(300 + step, "B"), (kk, n), 20)
        st, C = r.gemm_i64_oneshot(gpu_ctx, desc, A, B)
        assert st == r.SUCCESS, step
        np.testing.assert_array_equal(C, A @ B)


def test_oneshot_error_then_success(gpu_ctx):
    # a range error leaves the caller's buffer untouched and the next call is exact
    m, n, k = 64, 64, 64
    desc = r.gemm_desc(r.BOUNDED_U64, r.BOUND_GLOBAL_MAX_UNSIGNED, m, n, k, bound=1000)
    A = inputs.uint_range(inputs.operand_seed(7, "A"), (m, k), 10)
    B = inputs.uint_range(inputs.operand_seed(7, "B"), (k, n), 10)
    out = np.full((m, n), 9, dtype=np.uint64)
    st, _ = r.gemm_u64_oneshot(gpu_ctx, desc, A, B, out)
    assert st == r.RANGE_ERROR and (out == 9).all()
    small = (A % 2).astype(np.uint64), (B % 2).astype(np.uint64)
    st, C = r.gemm_u64_oneshot(gpu_ctx, desc, *small)
    assert st == r.SUCCESS
    np.testing.assert_array_equal(C, small[0] @ small[1])


@pytest.mark.parametrize("modulus,field", [(251, True), (256, False)])
def test_finite_oneshot_repeats(gpu_ctx, modulus, field):
    m, n, k = 100, 120, 140
    sem = r.FINITE_FIELD_U8 if field else r.FINITE_RING_U8
    desc = r.gemm_desc(sem, r.BOUND_NONE, m, n, k, finite_modulus=modulus)
    for step in range(3):
        A = inputs.bytes_below(400 + step, (m, k), modulus)
        B = inputs.bytes_below(500 + step, (k, n), modulus)
        st, C = r.gemm_finite_u8_oneshot(gpu_ctx, desc, modulus, A, B, field)
        assert st == r.SUCCESS
        np.testing.assert_array_equal(C, oracle.gemm_finite_u8(A, B, modulus))
