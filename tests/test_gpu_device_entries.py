"""The device-pointer pack entry points (rns8_mi355x_pack_*_device) and the
device-side magnitude proof of exact-wide packs.

* Bounded and finite device packs give the same planes as the host-array packs
  (and the oracle's), at ragged shapes and with a row stride above the width.
* An exact-wide device pack admits an operand iff 2 * max|x| < P (signed) or
  max x < P (unsigned) (reference exact_range.hpp:16-18 with the operand's own
  maximum): one element placed at the threshold, or one past it, anywhere in a
  matrix wider than one reduction block, decides the status.
"""
import ctypes

import numpy as np
import pytest

import oracle
import rns8_amd as r
from rns8_amd import hip, inputs

pytestmark = pytest.mark.gpu

P1 = 256
P8 = 13057518384392951040  # product of the first 8 ladder moduli


def _device_copy(arr):
    d = hip.malloc(arr.nbytes)
    hip.to_device(d, np.ascontiguousarray(arr))
    return d


def _pack_device(ctx, matrix, arr, ld, kind, modulus=0):
    d = _device_copy(arr)
    try:
        L = r.lib()
        if kind == "i64":
            st = L.rns8_mi355x_pack_i64_device(ctx.ptr, matrix.ptr, ctypes.c_void_p(d), ld, 0, None)
        elif kind == "u64":
            st = L.rns8_mi355x_pack_u64_device(ctx.ptr, matrix.ptr, ctypes.c_void_p(d), ld, 0, None)
        else:
            st = L.rns8_mi355x_pack_finite_u8_device(ctx.ptr, matrix.ptr, modulus, ctypes.c_void_p(d), ld, 0, None)
        hip.synchronize()
        return st
    finally:
        hip.free(d)


@pytest.mark.parametrize("rows,cols,ld", [(1, 1, 1), (37, 259, 300), (300, 4100, 4100)])
@pytest.mark.parametrize("kind", ["i64", "u64"])
def test_bounded_device_pack_matches_host_pack(gpu_ctx, rows, cols, ld, kind):
    sem = r.BOUNDED_I64 if kind == "i64" else r.BOUNDED_U64
    bk = r.BOUND_GLOBAL_MAX_ABS if kind == "i64" else r.BOUND_GLOBAL_MAX_UNSIGNED
    seed = rows * 7 + cols
    full = (inputs.full_int64(seed, (rows, ld)) if kind == "i64"
            else inputs.splitmix64(seed, rows * ld).reshape(rows, ld))
    dev = r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, sem, bk, 9))
    host = r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, sem, bk, 9))
    assert _pack_device(gpu_ctx, dev, full, ld, kind) == r.SUCCESS
    pack = r.pack_i64 if kind == "i64" else r.pack_u64
    assert pack(gpu_ctx, host, full, 1, ld=ld) == r.SUCCESS
    np.testing.assert_array_equal(dev.read_residues(), host.read_residues())
    opack = oracle.pack_i64 if kind == "i64" else oracle.pack_u64
    np.testing.assert_array_equal(dev.read_residues(), opack(np.ascontiguousarray(full[:, :cols]), 9))


@pytest.mark.parametrize("modulus,field", [(251, True), (256, False), (7, False)])
def test_finite_device_pack_matches_oracle(gpu_ctx, modulus, field):
    rows, cols, ld = 70, 1000, 1024
    sem = r.FINITE_FIELD_U8 if field else r.FINITE_RING_U8
    src = inputs.bytes_below(modulus, (rows, ld), 256)
    m = r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, sem, r.BOUND_NONE, 0))
    assert _pack_device(gpu_ctx, m, src, ld, "u8", modulus) == r.SUCCESS
    np.testing.assert_array_equal(m.read_residues(1)[0], oracle.pack_finite_u8(np.ascontiguousarray(src[:, :cols]),
                                                                              modulus))


@pytest.mark.parametrize("pos", [(0, 0), (299, 4999), (150, 2048), (7, 4095)])
def test_exact_wide_device_proof_threshold_signed(gpu_ctx, pos):
    rows, cols = 300, 5000
    base = inputs.int_range(11, (rows, cols), 20)
    for value, prefix, ok in [(P8 // 2 - 1, 8, True), (P8 // 2, 8, False), (-(P8 // 2 - 1), 8, True),
                              (-(P8 // 2), 8, False), (127, 1, True), (-128, 1, False), (-(1 << 63), 9, True)]:
        if prefix == 1:
            src = np.zeros((rows, cols), dtype=np.int64)
        else:
            src = base.copy()
        src[pos] = value
        m = r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, r.EXACT_WIDE_SIGNED, r.BOUND_NONE, prefix))
        st = _pack_device(gpu_ctx, m, src, cols, "i64")
        assert st == (r.SUCCESS if ok else r.RANGE_ERROR), (value, prefix, pos)


def test_exact_wide_device_proof_threshold_unsigned(gpu_ctx):
    rows, cols = 64, 3000
    for value, prefix, ok in [(P1 - 1, 1, True), (P1, 1, False), (P8 - 1, 8, True), (P8, 8, False)]:
        src = np.zeros((rows, cols), dtype=np.uint64)
        src[rows - 1, cols - 1] = np.uint64(value)
        m = r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, r.EXACT_WIDE_UNSIGNED, r.BOUND_NONE, prefix))
        st = _pack_device(gpu_ctx, m, src, cols, "u64")
        assert st == (r.SUCCESS if ok else r.RANGE_ERROR), (value, prefix)
