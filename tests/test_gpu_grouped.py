"""Grouped resident GEMM (rns8_gemm_rns_grouped / rns8_gemm_finite_u8_grouped)
through the C ABI.

Each task of a group must give exactly what an ungrouped rns8_gemm_rns /
rns8_gemm_finite_u8 gives for the same operands: residue planes byte for byte,
and the exported values equal the oracle's. Covered: bounded int64 and uint64,
split-K shapes, both tile configurations, finite field and ring moduli,
exact-wide limbs, groups above the 32 tasks of one launch, per-tile plans,
and the validation the reference applies (api_gemm.cpp:200-336,
hip_grouped_descriptor.cpp:474-512).
"""
import numpy as np
import pytest

import oracle
import rns8_amd as r
from rns8_amd import inputs

pytestmark = pytest.mark.gpu


class Group:
    """A plan, one (A, B, C, workspace) quadruple per task, and a reference C per task."""

    def __init__(self, ctx, desc, count, sem, tile_m=0, tile_n=0, prefix=None):
        self.ctx, self.plan = ctx, r.Plan(ctx, desc)
        p = self.plan.prefix if prefix is None else prefix
        bk = desc.bound_kind
        mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, bk, p, tile_m=tile_m, tile_n=tile_n))
        m, n, k = desc.m, desc.n, desc.k
        self.tasks = [(mk(m, k), mk(k, n), mk(m, n), r.Workspace(ctx, self.plan)) for _ in range(count)]
        self.refs = [mk(m, n) for _ in range(count)]
        self.prefix = p


def _pack_all(ctx, group, operands, sem, modulus=0):
    for i, ((A, B), (Am, Bm, _, _)) in enumerate(zip(operands, group.tasks)):
        if sem == r.BOUNDED_I64 or sem == r.EXACT_WIDE_SIGNED:
            r.check(r.pack_i64(ctx, Am, A, 2 * i + 1), "pack A")
            r.check(r.pack_i64(ctx, Bm, B, 2 * i + 2), "pack B")
        elif sem == r.BOUNDED_U64 or sem == r.EXACT_WIDE_UNSIGNED:
            r.check(r.pack_u64(ctx, Am, A, 2 * i + 1), "pack A")
            r.check(r.pack_u64(ctx, Bm, B, 2 * i + 2), "pack B")
        else:
            r.check(r.pack_finite_u8(ctx, Am, modulus, A, 2 * i + 1), "pack A")
            r.check(r.pack_finite_u8(ctx, Bm, modulus, B, 2 * i + 2), "pack B")


def _check_against_ungrouped(ctx, group, modulus=None):
    for (Am, Bm, Cm, ws), ref in zip(group.tasks, group.refs):
        if modulus is None:
            r.check(r.gemm_rns(ctx, group.plan, Am, Bm, ref, ws), "ungrouped gemm")
        else:
            r.check(r.gemm_finite_u8(ctx, group.plan, modulus, Am, Bm, ref, ws), "ungrouped gemm")
        np.testing.assert_array_equal(Cm.read_residues(), ref.read_residues())


@pytest.mark.parametrize("m,n,k,count", [(300, 200, 150, 5), (1024, 1024, 512, 2), (64, 64, 32, 40),
                                         (128, 128, 8192, 3), (33, 517, 70000, 2),
                                         (500, 7, 3000, 3), (8, 8, 80000, 2)])
def test_bounded_i64_group_matches_ungrouped_and_oracle(gpu_ctx, m, n, k, count):
    bound = 1 << 62
    desc = r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, m, n, k, bound=bound, max_prefix=9,
                       flags=r.PLAN_FORCE_FIXED_PREFIX)
    g = Group(gpu_ctx, desc, count, r.BOUNDED_I64)
    ops = [(inputs.int_range(inputs.operand_seed(50 + i, "A"), (m, k), 20),
            inputs.int_range(inputs.operand_seed(50 + i, "B"), (k, n), 20)) for i in range(count)]
    _pack_all(gpu_ctx, g, ops, r.BOUNDED_I64)
    r.check(r.gemm_rns_grouped(gpu_ctx, g.plan, g.tasks), "grouped gemm")
    # spot-check the first and last task against the oracle's export
    for i in (0, count - 1):
        out = np.zeros((m, n), dtype=np.int64)
        r.check(r.export_i64(gpu_ctx, g.plan, g.tasks[i][2], out), "export")
        rows = min(m, 16 if k < 10000 else 2)
        st, want = oracle.gemm_i64(ops[i][0], ops[i][1], 9, bound, row0=0, rows=rows)
        assert st == 0
        np.testing.assert_array_equal(out[:rows], want)
    _check_against_ungrouped(gpu_ctx, g)


def test_bounded_u64_group(gpu_ctx):
    m, n, k, count = 130, 257, 300, 3
    desc = r.gemm_desc(r.BOUNDED_U64, r.BOUND_GLOBAL_MAX_UNSIGNED, m, n, k, bound=(1 << 64) - 1)
    g = Group(gpu_ctx, desc, count, r.BOUNDED_U64)
    ops = [(inputs.uint_range(inputs.operand_seed(70 + i, "A"), (m, k), 27),
            inputs.uint_range(inputs.operand_seed(70 + i, "B"), (k, n), 27)) for i in range(count)]
    _pack_all(gpu_ctx, g, ops, r.BOUNDED_U64)
    r.check(r.gemm_rns_grouped(gpu_ctx, g.plan, g.tasks), "grouped gemm")
    for i in range(count):
        out = np.zeros((m, n), dtype=np.uint64)
        r.check(r.export_u64(gpu_ctx, g.plan, g.tasks[i][2], out), "export")
        want = (ops[i][0].astype(object) @ ops[i][1].astype(object))
        assert (out.astype(object) == want).all()
    _check_against_ungrouped(gpu_ctx, g)


@pytest.mark.parametrize("sem,modulus", [(r.FINITE_FIELD_U8, 251), (r.FINITE_RING_U8, 256), (r.FINITE_RING_U8, 7)])
def test_finite_group(gpu_ctx, sem, modulus):
    m, n, k, count = 200, 300, 1000, 4
    desc = r.gemm_desc(sem, r.BOUND_NONE, m, n, k, finite_modulus=modulus)
    g = Group(gpu_ctx, desc, count, sem, prefix=0)
    rng = np.random.default_rng(modulus)
    ops = [(rng.integers(0, modulus, size=(m, k), dtype=np.uint8), rng.integers(0, modulus, size=(k, n),
                                                                                   dtype=np.uint8))
           for _ in range(count)]
    _pack_all(gpu_ctx, g, ops, sem, modulus)
    r.check(r.gemm_finite_u8_grouped(gpu_ctx, g.plan, modulus, g.tasks), "grouped gemm")
    for i in range(count):
        out = np.zeros((m, n), dtype=np.uint8)
        r.check(r.export_finite_u8(gpu_ctx, g.plan, modulus, g.tasks[i][2], out), "export")
        want = (ops[i][0].astype(np.int64) @ ops[i][1].astype(np.int64)) % modulus
        np.testing.assert_array_equal(out, want.astype(np.uint8))
    _check_against_ungrouped(gpu_ctx, g, modulus)


def test_exact_wide_group(gpu_ctx):
    m, n, k, count = 70, 90, 40, 3
    desc = r.gemm_desc(r.EXACT_WIDE_SIGNED, r.BOUND_NONE, m, n, k, max_prefix=20, flags=r.PLAN_FORCE_FIXED_PREFIX)
    g = Group(gpu_ctx, desc, count, r.EXACT_WIDE_SIGNED)
    ops = [(inputs.full_int64(inputs.operand_seed(90 + i, "A"), (m, k)),
            inputs.full_int64(inputs.operand_seed(90 + i, "B"), (k, n))) for i in range(count)]
    _pack_all(gpu_ctx, g, ops, r.EXACT_WIDE_SIGNED)
    r.check(r.gemm_rns_grouped(gpu_ctx, g.plan, g.tasks), "grouped gemm")
    for i in range(count):
        out = np.zeros((m, n * 3), dtype=np.uint64)
        r.check(r.export_exact_wide_signed_limbs(gpu_ctx, g.plan, g.tasks[i][2], out, 3), "export")
        want = ops[i][0].astype(object) @ ops[i][1].astype(object)
        for row, col in [(0, 0), (m - 1, n - 1), (m // 2, 7), (3, n - 2)]:
            assert oracle.limbs_to_int(out[row, 3 * col:3 * col + 3], True) == want[row, col]
    _check_against_ungrouped(gpu_ctx, g)


def test_per_tile_group(gpu_ctx):
    # per-tile plans whose schedule selects several prefixes run the listed GEMM per task
    m, n, k, count = 200, 260, 9, 2
    rng = np.random.default_rng(8)
    A0 = [rng.integers(-(1 << 20), 1 << 20, size=(m, k)) for _ in range(count)]
    for A in A0:
        A[:64] >>= 18
    B0 = [rng.integers(-(1 << 20), 1 << 20, size=(k, n)) for _ in range(count)]
    ops = [(A.astype(np.int64), B.astype(np.int64)) for A, B in zip(A0, B0)]
    tc = -(-n // 64)
    bounds = [k << (22 if t // tc == 0 else 40) for t in range(-(-m // 64) * tc)]
    desc = r.gemm_desc(r.BOUNDED_I64, r.BOUND_PER_TILE_MAX_ABS, m, n, k, max_prefix=9, tile_m=64, tile_n=64,
                       tile_bounds=bounds)
    g = Group(gpu_ctx, desc, count, r.BOUNDED_I64, tile_m=64, tile_n=64)
    assert g.plan.schedule_info().prefix_group_count > 1
    _pack_all(gpu_ctx, g, ops, r.BOUNDED_I64)
    r.check(r.gemm_rns_grouped(gpu_ctx, g.plan, g.tasks), "grouped gemm")
    for i in range(count):
        out = np.zeros((m, n), dtype=np.int64)
        r.check(r.export_i64(gpu_ctx, g.plan, g.tasks[i][2], out), "export")
        np.testing.assert_array_equal(out, ops[i][0] @ ops[i][1])


def test_group_validation(gpu_ctx):
    m, n, k = 64, 80, 96
    desc = r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, m, n, k, bound=1 << 40)
    g = Group(gpu_ctx, desc, 3, r.BOUNDED_I64)
    ops = [(inputs.int_range(inputs.operand_seed(i, "A"), (m, k), 10),
            inputs.int_range(inputs.operand_seed(i, "B"), (k, n), 10)) for i in range(3)]
    _pack_all(gpu_ctx, g, ops, r.BOUNDED_I64)
    t = g.tasks
    assert r.gemm_rns_grouped(gpu_ctx, g.plan, t[:1]) == r.INVALID_ARGUMENT  # a group has at least two tasks
    assert r.gemm_rns_grouped(gpu_ctx, g.plan, [t[0], (t[0][0], t[1][1], t[1][2], t[1][3])]) == r.INVALID_ARGUMENT
    assert r.gemm_rns_grouped(gpu_ctx, g.plan, [t[0], (t[1][0], t[1][1], t[1][2], t[0][3])]) == r.INVALID_ARGUMENT
    # one task's result is another task's operand
    assert r.gemm_rns_grouped(gpu_ctx, g.plan, [t[0], (t[0][2], t[1][1], t[1][2], t[1][3])]) == r.INVALID_ARGUMENT
    # A == B inside a task
    assert r.gemm_rns_grouped(gpu_ctx, g.plan, [t[0], (t[1][0], t[1][0], t[1][2], t[1][3])]) == r.INVALID_ARGUMENT
    # a workspace made for another shape
    other = r.Plan(gpu_ctx, r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, m, n, k + 1, bound=1 << 40))
    ws_other = r.Workspace(gpu_ctx, other)
    assert r.gemm_rns_grouped(gpu_ctx, g.plan, [t[0], (t[1][0], t[1][1], t[1][2], ws_other)]) == \
        r.abi.WORKSPACE_TOO_SMALL
    # the valid group runs, and its contract is reported
    assert r.gemm_rns_grouped(gpu_ctx, g.plan, t) == r.SUCCESS
    st, info = r.grouped_contract_info(g.plan, 3)
    assert st == r.SUCCESS and info.public_execution_available == 1 and info.same_shape_required == 1
    assert info.output_domain == b"native_i64_u64_host"
    st, info = r.grouped_contract_info(g.plan, 1)
    assert st == r.SUCCESS and info.public_execution_available == 0
    assert info.unsupported_reason == b"task_count_must_exceed_one"
