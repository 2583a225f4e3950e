"""Every status expectation of tests/golden/reference_status_kats.json (the
reference's test_semantics_validation_cases.inc and test_api_validation_cases.inc)
through the C ABI on a live context: plans, matrices, contexts and oneshot
calls, with outputs checked untouched where a call is refused and exact where
it succeeds, and the two persistent finite sequences step by step."""
import ctypes as C

import numpy as np
import pytest

import rns8_amd as r
import status_kats as sk

pytestmark = pytest.mark.gpu

CASES = sk.KATS["cases"]


@pytest.mark.parametrize("case", CASES, ids=[c["ref"] for c in CASES])
def test_reference_status(gpu_ctx, case):
    assert sk.run_with_context(gpu_ctx, case) == sk.STATUS[case["expect"]], case["ref"]


def _finite_matrix(ctx, rows, cols, sem):
    return r.Matrix(ctx, r.matrix_desc(rows, cols, sem, r.BOUND_NONE, 0))


def test_persistent_finite_contracts(gpu_ctx):
    seq = sk.KATS["sequences"][0]
    m, n, k, lda, ldb, ldc = (seq[x] for x in ("m", "n", "k", "lda", "ldb", "ldc"))
    A = np.array(seq["A"], dtype=np.uint8).reshape(m, lda)
    B = np.array(seq["B"], dtype=np.uint8).reshape(k, ldb)
    want = seq["expect"]
    for sem_name, modulus in seq["moduli"]:
        sem = sk.NAMES[sem_name]
        desc = r.gemm_desc(sem, r.BOUND_NONE, m, n, k, finite_modulus=modulus)
        plan = r.Plan(gpu_ctx, desc)
        info = plan.schedule_info()
        for field, v in seq["schedule"].items():
            assert getattr(info, field) == v, field
        Am, Bm, Cm = (_finite_matrix(gpu_ctx, rr, cc, sem) for rr, cc in ((m, k), (k, n), (m, n)))
        ws = r.Workspace(gpu_ctx, plan)
        v1, v2 = seq["pack_versions"]
        assert r.pack_finite_u8(gpu_ctx, Am, modulus, A, v1, ld=lda) == sk.STATUS[want["pack"]]
        assert r.pack_finite_u8(gpu_ctx, Bm, modulus, B, v2, ld=ldb) == sk.STATUS[want["pack"]]
        assert r.gemm_finite_u8(gpu_ctx, plan, modulus, Am, Bm, Cm, ws) == sk.STATUS[want["gemm_finite_u8"]]
        out = np.full((m, ldc), seq["c_fill"], dtype=np.uint8)
        L = r.lib()
        st = L.rns8_export_finite_u8(gpu_ctx.ptr, plan.ptr, modulus, Cm.ptr, out.ctypes.data_as(C.c_void_p), ldc)
        assert st == sk.STATUS[want["export_finite_u8"]]
        flat = sk.exact_finite(seq["A"], seq["B"], lda, ldb, k, m, n, modulus, [seq["c_fill"]] * (m * ldc), ldc)
        assert out.reshape(-1).tolist() == flat
        wrong = np.zeros(m * ldc, dtype=np.uint64)
        assert L.rns8_export_u64(gpu_ctx.ptr, plan.ptr, Cm.ptr, wrong.ctypes.data_as(C.c_void_p),
                                 ldc) == sk.STATUS[want["export_u64"]]
        assert r.gemm_rns(gpu_ctx, plan, Am, Bm, Cm, ws) == sk.STATUS[want["gemm_rns"]]


def test_persistent_finite_modulus_mismatches(gpu_ctx):
    seq = sk.KATS["sequences"][1]
    ring, field = sk.NAMES["FINITE_RING_U8"], sk.NAMES["FINITE_FIELD_U8"]
    plan = r.Plan(gpu_ctx, r.gemm_desc(ring, r.BOUND_NONE, 1, 1, 1, finite_modulus=255))
    ws = r.Workspace(gpu_ctx, plan)
    Am, Bm, Cm = (_finite_matrix(gpu_ctx, 1, 1, ring) for _ in range(3))
    field_plan = r.Plan(gpu_ctx, r.gemm_desc(field, r.BOUND_NONE, 1, 1, 1, finite_modulus=251))
    Fm = _finite_matrix(gpu_ctx, 1, 1, field)
    A = np.array(seq["A"], dtype=np.uint8).reshape(1, 1)
    B = np.array(seq["B"], dtype=np.uint8).reshape(1, 1)
    out = np.zeros((1, 1), dtype=np.uint8)
    L = r.lib()
    for op, modulus, expect in seq["steps"]:
        if op == "export_finite_u8":
            st = L.rns8_export_finite_u8(gpu_ctx.ptr, plan.ptr, modulus, Cm.ptr, out.ctypes.data_as(C.c_void_p), 1)
        elif op == "pack_finite_u8_A":
            st = r.pack_finite_u8(gpu_ctx, Am, modulus, A, 1)
        elif op == "pack_finite_u8_B":
            st = r.pack_finite_u8(gpu_ctx, Bm, modulus, B, 1)
        elif op == "gemm_finite_u8":
            st = r.gemm_finite_u8(gpu_ctx, plan, modulus, Am, Bm, Cm, ws)
        else:
            st = r.pack_finite_u8(gpu_ctx, Fm, modulus, A, 1)
        assert st == sk.STATUS[expect], (op, modulus)
    assert out.reshape(-1).tolist() == seq["c_after"]
    assert field_plan.prefix == 0  # the field plan stays alive through the field pack
