"""The int64 / uint64 export at the 64-bit edges, through the C ABI.

Each value v is produced exactly as C = A x B with K = 2: A = [hi, lo],
B = [2^32, 1]^T, so v = hi * 2^32 + lo reaches beyond int64 (+-2^64 and
neighbours) while both operands stay in int64. Every value is exported on its
own (a 1 x 1 result), so each accept / reject decision is observed alone:
RANGE_ERROR exactly when |v| exceeds the contract's limit (min(bound, 2^63 - 1)
for v >= 0 and min(bound, 2^63) for v < 0 with int64; bound with uint64;
reference src/reconstruct/crt.cpp:113-129), the value itself otherwise.
Prefix 9 runs the 3-limb kernel, 10, 12 and 20 the 7-limb one. The same
decisions are checked on 1 x 256 results holding v in every cell, which at
prefixes 9..11 run the matrix-core export (results at least 256 columns wide).
"""
import numpy as np
import pytest

import rns8_amd as r

pytestmark = pytest.mark.gpu

TWO63 = 1 << 63
TWO64 = 1 << 64
EDGES = [0, 1, -1, TWO63 - 1, -TWO63, TWO63, -TWO63 - 1, TWO64 - 1, -TWO64 + 1, -TWO64, TWO64, TWO64 + 1,
         -TWO64 - 1, 1 << 65, -(1 << 65), (1 << 62) + 1, -(1 << 62) - 1, 1 << 62, -(1 << 62)]


def _split(v):
    hi, lo = divmod(v, 1 << 32)
    return hi, lo


def _export_one(ctx, sem, v, prefix, bound, width=1):
    hi, lo = _split(v)
    dt = np.uint64 if sem == r.BOUNDED_U64 else np.int64
    A = np.array([[hi, lo]], dtype=dt)
    B = np.repeat(np.array([[1 << 32], [1]], dtype=dt), width, axis=1)
    bk = r.BOUND_GLOBAL_MAX_UNSIGNED if sem == r.BOUNDED_U64 else r.BOUND_GLOBAL_MAX_ABS
    desc = r.gemm_desc(sem, bk, 1, width, 2, bound=bound, max_prefix=prefix, flags=r.PLAN_FORCE_FIXED_PREFIX)
    plan = r.Plan(ctx, desc)
    assert plan.prefix == prefix
    mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, bk, prefix))
    Am, Bm, Cm = mk(1, 2), mk(2, width), mk(1, width)
    ws = r.Workspace(ctx, plan)
    pack = r.pack_u64 if sem == r.BOUNDED_U64 else r.pack_i64
    r.check(pack(ctx, Am, A, 1), "pack A")
    r.check(pack(ctx, Bm, B, 2), "pack B")
    r.check(r.gemm_rns(ctx, plan, Am, Bm, Cm, ws), "gemm")
    out = np.zeros((1, width), dtype=dt)
    export = r.export_u64 if sem == r.BOUNDED_U64 else r.export_i64
    st = export(ctx, plan, Cm, out)
    if st == r.SUCCESS:
        assert len(set(out[0].tolist())) == 1, (v, out[0][:4])
    return st, int(out[0, 0])


@pytest.mark.parametrize("prefix,width", [(9, 1), (10, 1), (12, 1), (20, 1), (9, 256), (10, 256), (11, 256)])
@pytest.mark.parametrize("bound", [1 << 62, TWO63 - 1, TWO63])
def test_i64_export_edges(gpu_ctx, prefix, width, bound):
    for v in EDGES:
        st, got = _export_one(gpu_ctx, r.BOUNDED_I64, v, prefix, bound, width)
        limit = min(bound, TWO63 - 1) if v >= 0 else min(bound, TWO63)
        if abs(v) <= limit:
            assert st == r.SUCCESS, (v, bound)
            assert got == v, (v, bound)
        else:
            assert st == r.RANGE_ERROR, (v, bound)


@pytest.mark.parametrize("prefix,width", [(9, 1), (10, 1), (20, 1), (9, 256), (10, 256), (11, 256)])
@pytest.mark.parametrize("bound", [1 << 62, TWO63, TWO64 - 1])
def test_u64_export_edges(gpu_ctx, prefix, width, bound):
    for v in [x for x in EDGES if x >= 0]:
        st, got = _export_one(gpu_ctx, r.BOUNDED_U64, v, prefix, bound, width)
        if v <= bound:
            assert st == r.SUCCESS, (v, bound)
            assert got == v, (v, bound)
        else:
            assert st == r.RANGE_ERROR, (v, bound)
