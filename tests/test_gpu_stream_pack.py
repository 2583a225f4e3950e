"""GPU parity for packs whose planes exceed the 256 MB Infinity Cache.

Such packs store their planes with non-temporal stores (pack.hip), a path
no smaller test reaches. Every byte is checked: the planes of one large pack
must equal those of the same rows packed in bands small enough to take the
ordinary stores (themselves checked against the oracle by the other pack
tests), and sampled rows are compared with the oracle directly. The GEMV
case runs the full 8192 x 1 x 8192 bench shape (604 MB of A planes, whose
skinny GEMM loads are non-temporal too) against numpy's exact int64 product.
"""
import ctypes

import numpy as np
import pytest

import oracle
import rns8_amd as r
from rns8_amd import hip, inputs

pytestmark = pytest.mark.gpu

STREAM_BYTES = 256 << 20  # pack.hip kStreamPackBytes


def _pack_from(ctx, matrix, dptr, ld, kind):
    L = r.lib()
    fn = L.rns8_mi355x_pack_i64_device if kind == "i64" else L.rns8_mi355x_pack_u64_device
    st = fn(ctx.ptr, matrix.ptr, ctypes.c_void_p(dptr), ld, 0, None)
    hip.synchronize()
    return st


def _bands_match(ctx, src, sem, bk, prefix, kind, offset_bytes, band_rows):
    rows, cols = src.shape
    d = hip.malloc(src.nbytes + 16)
    try:
        base = d + offset_bytes
        hip.to_device(base, np.ascontiguousarray(src))
        big = r.Matrix(ctx, r.matrix_desc(rows, cols, sem, bk, prefix))
        assert prefix * rows * cols >= STREAM_BYTES
        assert _pack_from(ctx, big, base, cols, kind) == r.SUCCESS
        got = big.read_residues(prefix)
        del big
        for r0 in range(0, rows, band_rows):
            band = r.Matrix(ctx, r.matrix_desc(band_rows, cols, sem, bk, prefix))
            assert prefix * band_rows * cols < STREAM_BYTES
            assert _pack_from(ctx, band, base + r0 * cols * 8, cols, kind) == r.SUCCESS
            np.testing.assert_array_equal(got[:, r0:r0 + band_rows], band.read_residues(prefix), err_msg=f"rows {r0}+")
    finally:
        hip.free(d)
    opack = oracle.pack_i64 if kind == "i64" else oracle.pack_u64
    for row in (0, rows // 2 + 3, rows - 1):
        np.testing.assert_array_equal(got[:, row:row + 1], opack(src[row:row + 1], prefix), err_msg=f"row {row}")


@pytest.mark.parametrize("kind,offset", [("i64", 0), ("u64", 0), ("i64", 8)])
def test_streaming_pack_equals_band_packs(gpu_ctx, kind, offset):
    # 8192 x 4096 at 9 planes = 302 MB; offset 8 leaves the source 8-byte
    # aligned only, which takes the scalar-load variant
    rows, cols = 8192, 4096
    if kind == "i64":
        src, sem, bk = inputs.full_int64(8101, (rows, cols)), r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS
    else:
        src, sem, bk = inputs.splitmix64(8102, rows * cols).reshape(rows, cols), r.BOUNDED_U64, r.BOUND_GLOBAL_MAX_UNSIGNED
    _bands_match(gpu_ctx, src, sem, bk, 9, kind, offset, 2048)


def test_streaming_exact_wide_pack_equals_band_packs(gpu_ctx):
    # 4096 x 4096 at 20 planes = 335 MB: the variant that also proves max |x|
    src = inputs.full_int64(8103, (4096, 4096))
    _bands_match(gpu_ctx, src, r.EXACT_WIDE_SIGNED, r.BOUND_NONE, 20, "i64", 0, 1024)


def test_gemv_after_streaming_pack(gpu_ctx):
    m, k = 8192, 8192
    A = inputs.int_range(8104, (m, k), 20)
    B = inputs.int_range(8105, (k, 1), 20)
    desc = r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, m, 1, k, bound=k << 40, max_prefix=9,
                       flags=r.PLAN_FORCE_FIXED_PREFIX)
    plan = r.Plan(gpu_ctx, desc)
    assert plan.prefix == 9 and plan.selected_kernel().startswith("skinny_gemm_kernel")
    mk = lambda rows, cols: r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, 9))
    Am, Bm, Cm = mk(m, k), mk(k, 1), mk(m, 1)
    ws = r.Workspace(gpu_ctx, plan)
    r.check(r.pack_i64(gpu_ctx, Am, A, 1), "pack A")
    r.check(r.pack_i64(gpu_ctx, Bm, B, 2), "pack B")
    r.check(r.gemm_rns(gpu_ctx, plan, Am, Bm, Cm, ws), "gemm")
    out = np.zeros((m, 1), dtype=np.int64)
    r.check(r.export_i64(gpu_ctx, plan, Cm, out), "export")
    # |sum| < 8192 * 2^40 = 2^53: numpy's int64 product is exact
    np.testing.assert_array_equal(out, A @ B)
