"""rns8_mi355x_gemm_rns_noalloc (the GEMM entry point that allocates nothing)
against rns8_mi355x_gemm_rns_async, through the C ABI.

The no-allocation entry keeps split-K residues in the library's static
per-device scratch instead of a workspace. Its residue planes must equal the
workspace entry's byte for byte: on two calls in a row, the second on a
smaller shape that reuses (and only partly overwrites) the scratch the first
one filled; on a shape with no K split; and its refusals (split-K residues
beyond the 4 MiB scratch, exact-wide plans) must leave C as it was.
"""
import numpy as np
import pytest

import oracle
import rns8_amd as r
from rns8_amd import hip, inputs

pytestmark = pytest.mark.gpu


def _setup(ctx, signed, m, n, k, prefix, bound, seed):
    sem = r.BOUNDED_I64 if signed else r.BOUNDED_U64
    bk = r.BOUND_GLOBAL_MAX_ABS if signed else r.BOUND_GLOBAL_MAX_UNSIGNED
    plan = r.Plan(ctx, r.gemm_desc(sem, bk, m, n, k, bound=bound, max_prefix=prefix,
                                   flags=r.PLAN_FORCE_FIXED_PREFIX))
    Am = r.Matrix(ctx, r.matrix_desc(m, k, sem, bk, prefix))
    Bm = r.Matrix(ctx, r.matrix_desc(k, n, sem, bk, prefix))
    if signed:
        A = inputs.int_range(inputs.operand_seed(seed, "A"), (m, k), 20)
        B = inputs.int_range(inputs.operand_seed(seed, "B"), (k, n), 20)
        r.check(r.pack_i64(ctx, Am, A, 1), "pack A")
        r.check(r.pack_i64(ctx, Bm, B, 2), "pack B")
    else:
        A = inputs.uint_range(inputs.operand_seed(seed, "A"), (m, k), 23)
        B = inputs.uint_range(inputs.operand_seed(seed, "B"), (k, n), 23)
        r.check(r.pack_u64(ctx, Am, A, 1), "pack A")
        r.check(r.pack_u64(ctx, Bm, B, 2), "pack B")
    mk = lambda: r.Matrix(ctx, r.matrix_desc(m, n, sem, bk, prefix))  # noqa: E731
    return plan, Am, Bm, mk, A, B


def _noalloc(ctx, plan, Am, Bm, Cm):
    return r.lib().rns8_mi355x_gemm_rns_noalloc(ctx.ptr, plan.ptr, Am.ptr, Bm.ptr, Cm.ptr, None)


def _with_workspace(ctx, plan, Am, Bm):
    # on the context stream, after every earlier call there
    Cw = r.Matrix(ctx, r.matrix_desc(plan.desc.m, plan.desc.n, plan.desc.semantics, plan.desc.bound_kind,
                                     plan.prefix))
    ws = r.Workspace(ctx, plan)
    r.check(r.lib().rns8_mi355x_gemm_rns_async(ctx.ptr, plan.ptr, Am.ptr, Bm.ptr, Cw.ptr, ws.ptr, None), "gemm")
    hip.synchronize()
    return Cw


def test_noalloc_equals_workspace_entry_two_calls(gpu_ctx):
    ctx = gpu_ctx
    # call 1: the tall-skinny C5 shape, 16 K slices x 8 planes of 128 x 128
    # int8 residues = 2 MiB of scratch
    p1, A1, B1, mk1, _, _ = _setup(ctx, False, 128, 128, 65536, 8, 1 << 62, 1201)
    C1 = mk1()
    assert _noalloc(ctx, p1, A1, B1, C1) == r.SUCCESS
    # call 2, smaller: 96 x 80 x 20000 int64 at prefix 9 (4 slices, 276 KB of
    # the scratch); the first call's residues still fill the rest
    p2, A2, B2, mk2, A, B = _setup(ctx, True, 96, 80, 20000, 9, 1 << 62, 1202)
    C2 = mk2()
    assert _noalloc(ctx, p2, A2, B2, C2) == r.SUCCESS
    hip.synchronize()
    W1 = _with_workspace(ctx, p1, A1, B1)
    W2 = _with_workspace(ctx, p2, A2, B2)
    np.testing.assert_array_equal(C1.read_residues(), W1.read_residues())
    np.testing.assert_array_equal(C2.read_residues(), W2.read_residues())
    out = np.zeros((96, 80), dtype=np.int64)
    r.check(r.export_i64(ctx, p2, C2, out), "export")
    np.testing.assert_array_equal(out, oracle.exact_gemm_i64(A, B, limbs=1).view(np.int64))


def test_noalloc_without_split(gpu_ctx):
    """A shape whose GEMM runs without a K split uses no scratch."""
    ctx = gpu_ctx
    plan, Am, Bm, mk, _, _ = _setup(ctx, True, 300, 280, 1000, 9, 1 << 62, 1203)
    C = mk()
    assert _noalloc(ctx, plan, Am, Bm, C) == r.SUCCESS
    hip.synchronize()
    np.testing.assert_array_equal(C.read_residues(), _with_workspace(ctx, plan, Am, Bm).read_residues())


def test_noalloc_skinny_split(gpu_ctx):
    """A result 16 columns wide or less runs the skinny kernel; with a K split
    its residue slots live in the scratch (8 x 8 x 300000 at prefix 9: 62
    slices, 71 KB), after a larger split shape has filled more of it."""
    ctx = gpu_ctx
    p1, A1, B1, mk1, _, _ = _setup(ctx, True, 128, 128, 65536, 8, 1 << 62, 1205)
    assert _noalloc(ctx, p1, A1, B1, mk1()) == r.SUCCESS
    p2, A2, B2, mk2, A, B = _setup(ctx, True, 8, 8, 300000, 9, 1 << 62, 1206)
    C2 = mk2()
    assert _noalloc(ctx, p2, A2, B2, C2) == r.SUCCESS
    hip.synchronize()
    np.testing.assert_array_equal(C2.read_residues(), _with_workspace(ctx, p2, A2, B2).read_residues())


def test_noalloc_refusals_leave_result(gpu_ctx):
    """Split-K residues beyond the scratch (256 x 256 x 65536 at prefix 9: 15
    slices x 9 planes x 256 x 256 bytes = 8.8 MB) and exact-wide plans are
    refused before anything is enqueued; C keeps its earlier result."""
    ctx = gpu_ctx
    plan, Am, Bm, mk, _, _ = _setup(ctx, True, 256, 256, 65536, 9, 1 << 62, 1204)
    C = mk()
    W = _with_workspace(ctx, plan, Am, Bm)
    # C gets the product first through the workspace entry, then the refused call
    ws = r.Workspace(ctx, plan)
    r.check(r.lib().rns8_mi355x_gemm_rns_async(ctx.ptr, plan.ptr, Am.ptr, Bm.ptr, C.ptr, ws.ptr, None), "gemm")
    hip.synchronize()
    assert _noalloc(ctx, plan, Am, Bm, C) == r.abi.WORKSPACE_TOO_SMALL
    np.testing.assert_array_equal(C.read_residues(), W.read_residues())
    sem, bk = r.EXACT_WIDE_SIGNED, r.BOUND_NONE
    pw = r.Plan(ctx, r.gemm_desc(sem, bk, 4, 4, 4, max_prefix=18))
    mats = [r.Matrix(ctx, r.matrix_desc(4, 4, sem, bk, 18)) for _ in range(3)]
    for i, M in enumerate(mats[:2]):
        r.check(r.pack_i64(ctx, M, np.full((4, 4), 3 + i, dtype=np.int64), 10 + i), "pack")
    assert _noalloc(ctx, pw, mats[0], mats[1], mats[2]) == r.UNSUPPORTED_BACKEND
