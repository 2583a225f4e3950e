"""Source versions through the C ABI (reference src/core/api_pack.cpp:7-27 and
api_plan_workspace_fingerprint.inc:18-27).

A pack with a nonzero source version equal to the matrix's, into a matrix
whose residues are current, is skipped: the matrix keeps what the earlier
pack wrote, even if the caller passes different data (for finite matrices
the modulus must match as well). Version 0 never skips, a new version packs,
and a matrix nothing has written yet packs whatever the version. A GEMM
gives its result the version FNV-1a(A's version, B's version) (0 maps to 1),
and an exact-wide pack skipped this way keeps the earlier pack's proof.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
import rns8_amd as r
from rns8_amd import abi, inputs

pytestmark = pytest.mark.gpu


def _version(ctx, matrix):
    info = abi.new_struct(abi.ResidentLifetimeInfo)
    r.check(r.lib().rns8_get_resident_lifetime_info(matrix.ptr, None, None, 0, C.byref(info)), "lifetime info")
    return info.source_version


def _fnv(a, b):
    h = 1469598103934665603
    for v in (a, b):
        h = ((h ^ v) * 1099511628211) & (2**64 - 1)
    return h or 1


def test_bounded_pack_elision_and_gemm_version(gpu_ctx):
    m, k, n, p = 30, 40, 20, 9
    sem, bk = r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS
    mk = lambda rows, cols: r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, sem, bk, p))
    A = mk(m, k)
    X = inputs.int_range(1, (m, k), 30)
    Y = inputs.int_range(2, (m, k), 30)
    px, py = oracle.pack_i64(X, p), oracle.pack_i64(Y, p)

    r.check(r.pack_i64(gpu_ctx, A, X, 5), "first pack")  # nothing current yet: packs
    np.testing.assert_array_equal(A.read_residues(p), px)
    r.check(r.pack_i64(gpu_ctx, A, Y, 5), "same version")  # skipped: keeps X
    np.testing.assert_array_equal(A.read_residues(p), px)
    assert _version(gpu_ctx, A) == 5
    r.check(r.pack_i64(gpu_ctx, A, Y, 6), "new version")
    np.testing.assert_array_equal(A.read_residues(p), py)
    r.check(r.pack_i64(gpu_ctx, A, X, 0), "version 0")
    np.testing.assert_array_equal(A.read_residues(p), px)
    r.check(r.pack_i64(gpu_ctx, A, Y, 0), "version 0 again")  # 0 never skips
    np.testing.assert_array_equal(A.read_residues(p), py)

    # a matrix nothing has written packs whatever version it is given
    A2 = mk(m, k)
    r.check(r.pack_i64(gpu_ctx, A2, X, 6), "fresh matrix")
    np.testing.assert_array_equal(A2.read_residues(p), px)

    # the GEMM's result carries FNV-1a of its operands' versions
    Av = inputs.int_range(8, (m, k), 20)
    Bv = inputs.int_range(3, (k, n), 20)
    B = mk(k, n)
    r.check(r.pack_i64(gpu_ctx, B, Bv, 77), "pack B")
    r.check(r.pack_i64(gpu_ctx, A, Av, 41), "pack A")
    plan = r.Plan(gpu_ctx, r.gemm_desc(sem, bk, m, n, k, bound=1 << 62, max_prefix=p, flags=r.PLAN_FORCE_FIXED_PREFIX))
    Cm = mk(m, n)
    r.check(r.gemm_rns(gpu_ctx, plan, A, B, Cm, r.Workspace(gpu_ctx, plan)), "gemm")
    assert _version(gpu_ctx, Cm) == _fnv(41, 77)
    out = np.zeros((m, n), dtype=np.int64)
    r.check(r.export_i64(gpu_ctx, plan, Cm, out), "export")
    np.testing.assert_array_equal(out, Av @ Bv)


def test_finite_pack_elision_needs_the_same_modulus(gpu_ctx):
    m, k = 17, 33
    sem = r.FINITE_RING_U8
    A = r.Matrix(gpu_ctx, r.matrix_desc(m, k, sem, r.BOUND_NONE, 0))
    X = inputs.bytes_below(4, (m, k), 256)
    Y = inputs.bytes_below(5, (m, k), 256)
    r.check(r.pack_finite_u8(gpu_ctx, A, 97, X, 9), "first pack")
    np.testing.assert_array_equal(A.read_residues(1)[0], oracle.pack_finite_u8(X, 97).reshape(m, k))
    r.check(r.pack_finite_u8(gpu_ctx, A, 97, Y, 9), "same version and modulus")  # skipped
    np.testing.assert_array_equal(A.read_residues(1)[0], oracle.pack_finite_u8(X, 97).reshape(m, k))
    r.check(r.pack_finite_u8(gpu_ctx, A, 89, Y, 9), "same version, another modulus")  # packs
    np.testing.assert_array_equal(A.read_residues(1)[0], oracle.pack_finite_u8(Y, 89).reshape(m, k))


def test_exact_wide_same_version_keeps_the_proof(gpu_ctx):
    m, k, prefix = 12, 16, 20
    sem = r.EXACT_WIDE_SIGNED
    A = r.Matrix(gpu_ctx, r.matrix_desc(m, k, sem, r.BOUND_NONE, prefix))
    small = inputs.int_range(6, (m, k), 10)
    big = inputs.full_int64(7, (m, k))
    r.check(r.pack_i64(gpu_ctx, A, small, 3), "pack small")
    bound_small = A.exact_proof(gpu_ctx)[0]
    r.check(r.pack_i64(gpu_ctx, A, big, 3), "same version")  # skipped: residues and proof unchanged
    assert A.exact_proof(gpu_ctx)[0] == bound_small
    np.testing.assert_array_equal(A.read_residues(prefix), oracle.pack_i64(small, prefix))
    r.check(r.pack_i64(gpu_ctx, A, big, 4), "new version")
    assert A.exact_proof(gpu_ctx)[0] == max(abs(int(v)) for v in big.reshape(-1))
