"""Runs the reference's status expectations (tests/golden/reference_status_kats.json)
through the library's C ABI.

Each case is one call with the descriptor fields, arguments and expected
status the reference's validation tests hold, with the reference's own
backend ('OWN', CPU_REFERENCE there) mapped to the library's (HIP_DIRECT).
Without a device only the calls that need none are run: context options
refused before any device call, and plan validation through
rns8_mi355x_plan_schedule, which runs rns8_create_plan's validation,
routing and schedule without a context.
"""
from __future__ import annotations

import ctypes as C
import json
from pathlib import Path

import numpy as np

import rns8_amd as r
from rns8_amd import abi

KATS = json.loads((Path(__file__).parent / "golden" / "reference_status_kats.json").read_text())

I64MAX = (1 << 63) - 1
NAMES = {
    "I64MAX": I64MAX, "HUGE": I64MAX // 2 + 1, "U64MAX": (1 << 64) - 1,
    # rns8_semantics
    "BOUNDED_I64": 1, "BOUNDED_U64": 2, "EXACT_WIDE_SIGNED": 3, "EXACT_WIDE_UNSIGNED": 4, "WRAP_U64_MOD_2_64": 5,
    "FINITE_RING_U8": 6, "FINITE_FIELD_U8": 7,
    # rns8_bound_kind
    "NONE": 0, "GLOBAL_MAX_ABS": 1, "GLOBAL_MAX_UNSIGNED": 2, "PER_TILE_MAX_ABS": 3, "PER_TILE_MAX_UNSIGNED": 4,
    # rns8_layout
    "ROW_MAJOR": 1, "COLUMN_MAJOR": 2,
    # rns8_backend_kind: the reference's own backend is this library's
    "OWN": 2, "HIPBLASLT": 3, "CK": 4, "ROCWMMA": 5, "WRAP64_BYTE_LIMB": 6,
}
STATUS = {"SUCCESS": 0, "INVALID_ARGUMENT": 1, "UNSUPPORTED_BACKEND": 4, "RANGE_ERROR": 5}


def value(v):
    return NAMES[v] if isinstance(v, str) else v


def gemm_desc(fields: dict):
    d = abi.new_struct(abi.GemmDesc)
    keep = {}
    for key, v in fields.items():
        if key == "tile_bounds":
            arr = (C.c_uint64 * len(v))(*v)
            keep["tile_bounds"] = arr
            d.tile_bounds = C.cast(arr, C.POINTER(C.c_uint64))
            if "tile_bounds_count" not in fields:
                d.tile_bounds_count = len(v)
        else:
            setattr(d, key, value(v))
    return d, keep


def matrix_desc(fields: dict):
    d = abi.new_struct(abi.MatrixDesc)
    for key, v in fields.items():
        setattr(d, key, value(v))
    return d


def context_options(fields: dict):
    o = abi.new_struct(abi.ContextOptions)
    for key, v in fields.items():
        setattr(o, key, value(v))
    return o


def device_free(case: dict) -> bool:
    """Calls whose expected status is reached before any device call."""
    if case["call"] == "create_plan":
        return True
    return case["call"] == "create_context" and case["expect"] != "SUCCESS"


def run_device_free(case: dict) -> int:
    L = r.lib()
    if case["call"] == "create_context":
        out = C.c_void_p()
        st = L.rns8_create_context(case["device"], C.byref(context_options(case["options"])), C.byref(out))
        if case.get("out_null"):
            assert not out.value, case["ref"]
        return st
    desc, _keep = gemm_desc(case["desc"])
    info = abi.new_struct(abi.PlanScheduleInfo)
    written = C.c_uint64(0)
    return L.rns8_mi355x_plan_schedule(C.byref(desc), C.byref(info), None, 0, C.byref(written))


ONESHOT = {
    "gemm_i64_oneshot": ("rns8_gemm_i64_oneshot", np.int64, False),
    "gemm_u64_oneshot": ("rns8_gemm_u64_oneshot", np.uint64, False),
    "gemm_finite_ring_u8_oneshot": ("rns8_gemm_finite_ring_u8_oneshot", np.uint8, True),
    "gemm_finite_field_u8_oneshot": ("rns8_gemm_finite_field_u8_oneshot", np.uint8, True),
}


def exact_finite(A, B, lda, ldb, k, m, n, modulus, C_before, ldc):
    """Expected C of a finite oneshot: the product mod `modulus` in its cells,
    every other byte of C as it was (reference test_semantics_support.inc:
    52-70)."""
    out = list(C_before)
    for row in range(m):
        for col in range(n):
            acc = 0
            for kk in range(k):
                acc = (acc + (A[row * lda + kk] % modulus) * (B[kk * ldb + col] % modulus)) % modulus
            out[row * ldc + col] = acc
    return out


def run_with_context(ctx, case: dict) -> int:
    """Any case, on a live context (device required)."""
    L = r.lib()
    call = case["call"]
    if call == "create_context":
        return run_device_free(case)
    if call == "create_plan":
        desc, _keep = gemm_desc(case["desc"])
        out = C.c_void_p()
        st = L.rns8_create_plan(ctx.ptr, C.byref(desc), C.byref(out))
        if case.get("out_null"):
            assert not out.value, case["ref"]
        if out.value:
            L.rns8_destroy_plan(out)
        return st
    if call == "create_matrix":
        desc = matrix_desc(case["desc"])
        out = C.c_void_p()
        st = L.rns8_create_matrix(ctx.ptr, C.byref(desc), C.byref(out))
        if case.get("out_null"):
            assert not out.value, case["ref"]
        if out.value:
            L.rns8_destroy_matrix(out)
        return st
    name, dt, finite = ONESHOT[call]
    desc, _keep = gemm_desc(case["desc"])
    A = np.array(case["A"], dtype=dt)
    B = np.array(case["B"], dtype=dt)
    Cb = np.array(case["C"], dtype=dt)
    Cout = Cb.copy()
    ptr = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    lda, ldb, ldc = value(case["lda"]), value(case["ldb"]), value(case["ldc"])
    fn = getattr(L, name)
    if finite:
        st = fn(ctx.ptr, C.byref(desc), case["modulus"], ptr(A), lda, ptr(B), ldb, ptr(Cout), ldc)
    else:
        st = fn(ctx.ptr, C.byref(desc), ptr(A), lda, ptr(B), ldb, ptr(Cout), ldc)
    want = case.get("c_after")
    if want == "exact_finite":
        d = case["desc"]
        want = exact_finite(case["A"], case["B"], lda, ldb, d["k"], d["m"], d["n"], case["modulus"], case["C"], ldc)
    if want is not None:
        assert Cout.tolist() == np.array(want, dtype=dt).tolist(), case["ref"]
    return st
