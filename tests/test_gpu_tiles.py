"""Per-tile bounded schedules on the GPU, through the C ABI, against the oracle.

The plan's schedule drives a listed GEMM (planes below each tile's selected
prefix, zero-output tiles filled with 0, higher planes untouched) and a
per-tile export (each tile with its own prefix and bound). Checks:
- the reference's per-tile oneshot KATs (tests/golden/reference_tile_kats.json,
  from test_bounded_gemm_per_tile_cases.inc): status, exact products, and the
  caller's buffer untouched on RANGE_ERROR;
- random per-tile bounds set from the true per-tile maxima at every schedule
  tile size: exported values equal the exact products, residue planes equal
  the oracle's tiled GEMM byte for byte, including the sentinel bytes of the
  planes no tile computes;
- a tile bound one below its true maximum is a RANGE_ERROR;
- zero-output tiles (bound 0 with the opt-in) export 0 whatever A x B holds;
- a collapsed schedule (every tile at the plan prefix) still checks each
  tile's own bound;
- K above the int32-safe block (accumulating launches of the listed GEMM).
"""
import ctypes
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
import rns8_amd as r
from rns8_amd import hip

pytestmark = pytest.mark.gpu

KATS = json.loads((Path(__file__).parent / "golden" / "reference_tile_kats.json").read_text())
SENTINEL = -91


def _kinds(signed):
    if signed:
        return r.BOUNDED_I64, r.abi.BOUND_PER_TILE_MAX_ABS, np.int64
    return r.BOUNDED_U64, r.abi.BOUND_PER_TILE_MAX_UNSIGNED, np.uint64


def _tile_run(ctx, signed, A, B, tile_m, tile_n, bounds, budget=9, flags=0, device_export=False):
    """Plan, pack, GEMM (C pre-filled with SENTINEL bytes) and export; returns
    (gemm status, export status, exported values, C residue planes, plan prefix)."""
    sem, bk, dt = _kinds(signed)
    m, k = A.shape
    n = B.shape[1]
    desc = r.gemm_desc(sem, bk, m, n, k, max_prefix=budget, flags=flags, tile_m=tile_m, tile_n=tile_n,
                       tile_bounds=bounds)
    plan = r.Plan(ctx, desc)
    sp = plan.prefix
    mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, bk, sp, tile_m=tile_m, tile_n=tile_n))
    Am, Bm, Cm = mk(m, k), mk(k, n), mk(m, n)
    ws = r.Workspace(ctx, plan)
    pack = r.pack_i64 if signed else r.pack_u64
    r.check(pack(ctx, Am, A, 1), "pack A")
    r.check(pack(ctx, Bm, B, 2), "pack B")
    ptr, _, pitch, count = Cm.planes()
    hip.memset(ptr, SENTINEL & 0xFF, pitch * count)
    hip.synchronize()
    gst = r.gemm_rns(ctx, plan, Am, Bm, Cm, ws)
    out = np.full((m, n), 77, dtype=dt)
    if gst != r.SUCCESS:
        return gst, None, out, None, sp
    if device_export:
        d_out = hip.malloc(out.nbytes)
        d_status = hip.malloc(4)
        try:
            hip.to_device(d_out, out)
            hip.memset(d_status, 0, 4)
            fn = r.lib().rns8_mi355x_export_i64_device if signed else r.lib().rns8_mi355x_export_u64_device
            r.check(fn(ctx.ptr, plan.ptr, Cm.ptr, ctypes.c_void_p(d_out), n, ctypes.c_void_p(d_status), None),
                    "device export")
            hip.synchronize()
            status = np.zeros(1, dtype=np.uint32)
            hip.from_device(status, d_status)
            hip.from_device(out, d_out)
            est = r.SUCCESS if status[0] == 0 else r.RANGE_ERROR
        finally:
            hip.free(d_out)
            hip.free(d_status)
    else:
        est = (r.export_i64 if signed else r.export_u64)(ctx, plan, Cm, out)
    return gst, est, out, Cm.read_residues(sp), sp


def _oracle_planes(signed, A, B, tile_m, tile_n, bounds, budget=9, flags=0):
    st, entries, summary = oracle.tile_schedule(signed, A.shape[0], B.shape[1], tile_m, tile_n, bounds, budget, flags)
    assert st == 0
    sp = summary.max_selected
    pack = oracle.pack_i64 if signed else oracle.pack_u64
    Cp = np.full((sp, A.shape[0], B.shape[1]), SENTINEL, dtype=np.int8)
    Cp = oracle.gemm_rns_tiled(pack(A, sp), pack(B, sp), Cp, entries)
    ost, oout = oracle.export_tiled(Cp, tile_m, tile_n, entries, bounds, signed)
    return Cp, ost, oout, sp


@pytest.mark.parametrize("case", KATS["oneshots"], ids=lambda c: c["name"])
def test_reference_oneshot_kats(gpu_ctx, case):
    m, n, k = case["m"], case["n"], case["k"]
    sem, bk, dt = _kinds(case["signed"])
    a, b = case["a_col"], case["b_row"]
    A = np.array([[a["lo"] if i < a["split"] else a["hi"]] for i in range(m)], dtype=dt)
    B = np.array([[b["lo"] if j < b["split"] else b["hi"] for j in range(n)]], dtype=dt)
    desc = r.gemm_desc(sem, bk, m, n, k, max_prefix=9, flags=case["flags"], tile_m=case["tile"],
                       tile_n=case["tile"], tile_bounds=case["bounds"])
    out = np.full((m, n), 5, dtype=dt)
    oneshot = r.gemm_i64_oneshot if case["signed"] else r.gemm_u64_oneshot
    st, got = oneshot(gpu_ctx, desc, A, B, out)
    assert st == case["status"]
    if st == r.SUCCESS:
        want = np.array([[int(A[i, 0]) * int(B[0, j]) for j in range(n)] for i in range(m)], dtype=object)
        assert (got.astype(object) == want).all()
    else:
        assert (got == 5).all()  # caller's buffer untouched


def _tiled_operands(rng, signed, m, n, k):
    # per-row / per-column magnitudes, so tiles need very different prefixes
    dt = np.int64 if signed else np.uint64
    row_bits = rng.integers(1, 29, size=m)
    col_bits = rng.integers(1, 29, size=n)
    A = np.zeros((m, k), dtype=object)
    B = np.zeros((k, n), dtype=object)
    for i in range(m):
        v = rng.integers(0, 1 << int(row_bits[i]), size=k)
        s = np.where(rng.random(k) < 0.5, -1, 1) if signed else np.ones(k, dtype=np.int64)
        A[i] = [int(x) * int(y) for x, y in zip(v, s)]
    for j in range(n):
        B[:, j] = [int(x) for x in rng.integers(0, 1 << int(col_bits[j]), size=k)]
    return A.astype(dt), B.astype(dt)


def _tile_maxima(exact, tile_m, tile_n):
    m, n = exact.shape
    tr, tc = -(-m // tile_m), -(-n // tile_n)
    return [int(max(abs(int(x)) for x in exact[(t // tc) * tile_m:(t // tc + 1) * tile_m,
                                                (t % tc) * tile_n:(t % tc + 1) * tile_n].flat))
            for t in range(tr * tc)]


@pytest.mark.parametrize("tile_m,tile_n", [(64, 64), (128, 128), (64, 256), (512, 128), (256, 512)])
@pytest.mark.parametrize("signed", [True, False])
def test_random_tiles_match_oracle(gpu_ctx, tile_m, tile_n, signed):
    rng = np.random.default_rng(tile_m * 7 + tile_n + signed)
    m, n, k = int(rng.integers(300, 700)), int(rng.integers(300, 700)), int(rng.integers(1, 24))
    A, B = _tiled_operands(rng, signed, m, n, k)
    exact = A.astype(object) @ B.astype(object)
    bounds = _tile_maxima(exact, tile_m, tile_n)
    gst, est, out, planes, sp = _tile_run(gpu_ctx, signed, A, B, tile_m, tile_n, bounds)
    assert gst == r.SUCCESS and est == r.SUCCESS
    assert (out.astype(object) == exact).all()
    Cp, ost, oout, osp = _oracle_planes(signed, A, B, tile_m, tile_n, bounds)
    assert sp == osp and ost == 0
    np.testing.assert_array_equal(planes, Cp)  # includes untouched sentinel planes
    np.testing.assert_array_equal(out, oout)


def _block_operands(rng, signed, m, n, k, block=64):
    # magnitudes set per 64-row block of A and per 64-column block of B, so the
    # quadrants of one GEMM unit need different prefixes; |C| < 24 * 2^56 fits int64
    dt = np.int64 if signed else np.uint64
    rb = np.repeat(rng.integers(1, 29, size=-(-m // block)), block)[:m]
    cb = np.repeat(rng.integers(1, 29, size=-(-n // block)), block)[:n]
    A = rng.integers(0, 1 << 28, size=(m, k)) >> (28 - rb[:, None])
    B = rng.integers(0, 1 << 28, size=(k, n)) >> (28 - cb[None, :])
    if signed:
        A = A * np.where(rng.random((m, k)) < 0.5, -1, 1)
    return A.astype(dt), B.astype(dt)


def _tile_maxima_np(exact, tile_m, tile_n):
    mag = np.abs(exact) if exact.dtype == np.int64 else exact
    rows = np.maximum.reduceat(mag, np.arange(0, mag.shape[0], tile_m), axis=0)
    return [int(x) for x in np.maximum.reduceat(rows, np.arange(0, mag.shape[1], tile_n), axis=1).reshape(-1)]


def _units_at_edge(entries, m, n, tile_m, tile_n, planes, edge):
    # (plane, edge x edge tile) pairs with some quadrant whose schedule tile selects more than the plane
    sel = {(e.tile_row, e.tile_col): e.selected_prefix for e in entries}
    count = 0
    for p in range(planes):
        for r0 in range(0, m, edge):
            for c0 in range(0, n, edge):
                quads = [(r0 + dr, c0 + dc) for dr in (0, edge // 2) for dc in (0, edge // 2)
                         if r0 + dr < m and c0 + dc < n]
                count += any(sel[(qr // tile_m, qc // tile_n)] > p for qr, qc in quads)
    return count


@pytest.mark.parametrize("tile_m,tile_n", [(128, 128), (256, 128), (512, 256)])
@pytest.mark.parametrize("signed", [True, False])
def test_large_units_match_oracle(gpu_ctx, tile_m, tile_n, signed):
    # enough 256 x 256 units that the listed GEMM runs its large configuration
    rng = np.random.default_rng(100 + tile_m + tile_n + signed)
    m, n, k = 1900 + int(rng.integers(0, 100)), 1800 + int(rng.integers(0, 100)), int(rng.integers(8, 24))
    A, B = _block_operands(rng, signed, m, n, k)
    exact = A @ B
    bounds = _tile_maxima_np(exact, tile_m, tile_n)
    st, entries, summary = oracle.tile_schedule(signed, m, n, tile_m, tile_n, bounds, 9, 0)
    assert st == 0 and summary.group_count > 1
    assert _units_at_edge(entries, m, n, tile_m, tile_n, summary.max_selected, 256) >= 256
    gst, est, out, planes, sp = _tile_run(gpu_ctx, signed, A, B, tile_m, tile_n, bounds)
    assert gst == r.SUCCESS and est == r.SUCCESS
    np.testing.assert_array_equal(out, exact)
    Cp, ost, oout, osp = _oracle_planes(signed, A, B, tile_m, tile_n, bounds)
    assert sp == osp and ost == 0
    np.testing.assert_array_equal(planes, Cp)


@pytest.mark.parametrize("signed", [True, False])
def test_tile_bound_one_below_maximum_is_range_error(gpu_ctx, signed):
    rng = np.random.default_rng(40 + signed)
    m, n, k = 200, 330, 9
    A, B = _tiled_operands(rng, signed, m, n, k)
    exact = A.astype(object) @ B.astype(object)
    bounds = _tile_maxima(exact, 64, 128)
    # the tile with the largest maximum, and one from the middle
    for hot in {int(np.argmax(bounds)), len(bounds) // 2}:
        if bounds[hot] == 0:
            continue
        low = list(bounds)
        low[hot] -= 1
        gst, est, out, _, _ = _tile_run(gpu_ctx, signed, A, B, 64, 128, low)
        assert gst == r.SUCCESS and est == r.RANGE_ERROR
        assert (out == 77).all()  # host export leaves the buffer untouched


def test_zero_output_tiles(gpu_ctx):
    # bound 0 with the opt-in flag: the tile exports 0 and its planes are 0,
    # whatever the product holds there (the bound is the caller's proof)
    rng = np.random.default_rng(3)
    m, n, k = 190, 260, 5
    A = rng.integers(-1000, 1000, size=(m, k)).astype(np.int64)
    B = rng.integers(-1000, 1000, size=(k, n)).astype(np.int64)
    A[64:128] = 0  # tile row 1 has a true zero product
    exact = A.astype(object) @ B.astype(object)
    bounds = _tile_maxima(exact, 64, 64)
    tc = -(-n // 64)
    zero_tiles = [tc + 1, tc + 2, 0, 2 * tc + 3]  # two true zeros, two with non-zero products
    for t in zero_tiles:
        bounds[t] = 0
    flags = r.abi.PLAN_ALLOW_PROVEN_ZERO_TILE_SKIPS
    gst, est, out, planes, sp = _tile_run(gpu_ctx, True, A, B, 64, 64, bounds, flags=flags)
    assert gst == r.SUCCESS and est == r.SUCCESS
    Cp, ost, oout, osp = _oracle_planes(True, A, B, 64, 64, bounds, flags=flags)
    assert ost == 0 and sp == osp
    np.testing.assert_array_equal(planes, Cp)
    np.testing.assert_array_equal(out, oout)
    for t in zero_tiles:
        r0, c0 = (t // tc) * 64, (t % tc) * 64
        assert not out[r0:r0 + 64, c0:c0 + 64].any()


def test_collapsed_schedule_checks_tile_bounds(gpu_ctx):
    # every tile requires the budget (8), so the schedule collapses and the
    # ordinary GEMM runs; the export still uses each tile's own bound
    rng = np.random.default_rng(11)
    m, n, k = 300, 200, 17
    A = rng.integers(1 << 27, 1 << 28, size=(m, k)) * np.where(rng.random((m, k)) < 0.5, -1, 1)
    B = rng.integers(1 << 27, 1 << 28, size=(k, n))
    exact = A.astype(object) @ B.astype(object)
    bounds = _tile_maxima(exact, 128, 128)
    st, _, summary = oracle.tile_schedule(True, m, n, 128, 128, bounds, 8, 0)
    assert st == 0 and summary.collapsed == 1
    gst, est, out, planes, sp = _tile_run(gpu_ctx, True, A, B, 128, 128, bounds, budget=8)
    assert sp == 8 and gst == r.SUCCESS and est == r.SUCCESS
    assert (out.astype(object) == exact).all()
    low = list(bounds)
    low[1] -= 1
    gst, est, out, _, _ = _tile_run(gpu_ctx, True, A, B, 128, 128, low, budget=8)
    assert gst == r.SUCCESS and est == r.RANGE_ERROR
    assert (out == 77).all()


@pytest.mark.parametrize("m,n,k", [(8, 8, 100000), (8192, 1, 8192)])
def test_collapsed_schedule_narrow_split_k(gpu_ctx, m, n, k):
    # Every tile at the budget collapses the schedule, so the ordinary GEMM
    # runs: for results at most 16 columns wide the skinny kernel, which
    # splits K into int8 residue slots here (100000 > 65536; 8192 rows at 9
    # planes). The plan sizes that workspace like a global plan, and
    # rns8_gemm_rns, the grouped entry and the no-allocation entry all export
    # the exact product.
    ctx = gpu_ctx
    sem, bk, _ = _kinds(True)
    tile = 128
    tiles = ((m + tile - 1) // tile) * ((n + tile - 1) // tile)
    bounds = [(1 << 63) - 1] * tiles  # 2 * bound > P8: every tile requires prefix 9
    st, _, summary = oracle.tile_schedule(True, m, n, tile, tile, bounds, 9, 0)
    assert st == 0 and summary.collapsed == 1
    plan = r.Plan(ctx, r.gemm_desc(sem, bk, m, n, k, max_prefix=9, tile_m=tile, tile_n=tile, tile_bounds=bounds))
    assert plan.prefix == 9
    assert "skinny_gemm_kernel" in plan.selected_kernel() and "K split" in plan.selected_kernel()
    assert plan.backend_info().workspace_required_bytes > 0
    rng = np.random.default_rng(m + k)
    ops = [(rng.integers(-(1 << 20), 1 << 20, size=(m, k)).astype(np.int64),
            rng.integers(-(1 << 20), 1 << 20, size=(k, n)).astype(np.int64)) for _ in range(2)]
    mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, bk, 9, tile_m=tile, tile_n=tile))  # noqa: E731
    packed = []
    for i, (A, B) in enumerate(ops):
        Am, Bm = mk(m, k), mk(k, n)
        r.check(r.pack_i64(ctx, Am, A, 10 + 2 * i), "pack A")
        r.check(r.pack_i64(ctx, Bm, B, 11 + 2 * i), "pack B")
        packed.append((Am, Bm))

    def export(Cm, want):
        out = np.full((m, n), 77, dtype=np.int64)
        assert r.export_i64(ctx, plan, Cm, out) == r.SUCCESS
        np.testing.assert_array_equal(out, want)

    exact = [A @ B for A, B in ops]  # |C| < 2^54: exact in int64
    Am, Bm = packed[0]
    C1, ws1 = mk(m, n), r.Workspace(ctx, plan)
    assert r.gemm_rns(ctx, plan, Am, Bm, C1, ws1) == r.SUCCESS
    export(C1, exact[0])
    Cg = [mk(m, n), mk(m, n)]
    wsg = [r.Workspace(ctx, plan), r.Workspace(ctx, plan)]
    trip = [(packed[i][0], packed[i][1], Cg[i], wsg[i]) for i in range(2)]
    assert r.gemm_rns_grouped(ctx, plan, trip) == r.SUCCESS
    for i in range(2):
        export(Cg[i], exact[i])
    Cn = mk(m, n)
    Am, Bm = packed[1]
    assert r.lib().rns8_mi355x_gemm_rns_noalloc(ctx.ptr, plan.ptr, Am.ptr, Bm.ptr, Cn.ptr, None) == r.SUCCESS
    hip.synchronize()
    export(Cn, exact[1])


@pytest.mark.parametrize("signed", [True, False])
def test_device_export_matches_host_export(gpu_ctx, signed):
    rng = np.random.default_rng(21 + signed)
    m, n, k = 257, 131, 6
    A, B = _tiled_operands(rng, signed, m, n, k)
    exact = A.astype(object) @ B.astype(object)
    bounds = _tile_maxima(exact, 128, 64)
    gst, est, out, _, _ = _tile_run(gpu_ctx, signed, A, B, 128, 64, bounds, device_export=True)
    assert gst == r.SUCCESS and est == r.SUCCESS
    assert (out.astype(object) == exact).all()


def test_k_above_int32_block(gpu_ctx):
    # K = 70000: two accumulating launches of the listed GEMM
    rng = np.random.default_rng(5)
    m, n, k = 140, 200, 70000
    A = rng.integers(-1024, 1025, size=(m, k)).astype(np.int64)
    B = rng.integers(-1024, 1025, size=(k, n)).astype(np.int64)
    B[:, 64:128] //= 1024  # a column block with a smaller prefix
    exact = A @ B  # |C| < 2^37: exact in int64
    bounds = _tile_maxima(exact.astype(object), 64, 64)
    gst, est, out, planes, sp = _tile_run(gpu_ctx, True, A, B, 64, 64, bounds)
    assert gst == r.SUCCESS and est == r.SUCCESS
    np.testing.assert_array_equal(out, exact)


def test_zero_row_col_proofs_and_unsigned_zero_tiles(gpu_ctx):
    # proof masks flag the tiles they touch (the GEMM still computes them) and
    # uint64 zero-output tiles export 0
    rng = np.random.default_rng(17)
    m, n, k = 200, 190, 7
    A = rng.integers(0, 1 << 20, size=(m, k)).astype(np.uint64)
    B = rng.integers(0, 1 << 20, size=(k, n)).astype(np.uint64)
    A[5] = 0
    B[:, 70] = 0
    exact = A.astype(object) @ B.astype(object)
    bounds = _tile_maxima(exact, 64, 64)
    tc = -(-n // 64)
    bounds[tc + 1] = 0  # zero-output tile (its product is not zero)
    za = np.zeros(m, dtype=np.uint8)
    zb = np.zeros(n, dtype=np.uint8)
    za[5] = 1
    zb[70] = 1
    flags = r.abi.PLAN_ALLOW_PROVEN_ZERO_TILE_SKIPS | r.abi.PLAN_ALLOW_PROVEN_ZERO_ROW_COL_SKIPS
    sem, bk, dt = _kinds(False)
    desc = r.gemm_desc(sem, bk, m, n, k, max_prefix=9, flags=flags, tile_m=64, tile_n=64, tile_bounds=bounds,
                       zero_a_rows=za, zero_b_cols=zb)
    plan = r.Plan(gpu_ctx, desc)
    entries = plan.tile_schedule()
    assert any(e.flags & 2 for e in entries) and entries[tc + 1].flags & 1
    st, oentries, summary = oracle.tile_schedule(False, m, n, 64, 64, bounds, 9, flags, za, zb)
    assert st == 0 and [e.flags for e in entries] == [e.flags for e in oentries]
    sp = plan.prefix
    mk = lambda rows, cols: r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, sem, bk, sp, tile_m=64, tile_n=64))
    Am, Bm, Cm = mk(m, k), mk(k, n), mk(m, n)
    ws = r.Workspace(gpu_ctx, plan)
    r.check(r.pack_u64(gpu_ctx, Am, A, 1), "pack A")
    r.check(r.pack_u64(gpu_ctx, Bm, B, 2), "pack B")
    r.check(r.gemm_rns(gpu_ctx, plan, Am, Bm, Cm, ws), "gemm")
    out = np.full((m, n), 3, dtype=np.uint64)
    assert r.export_u64(gpu_ctx, plan, Cm, out) == r.SUCCESS
    want = exact.copy()
    r0, c0 = 64, 64
    want[r0:r0 + 64, c0:c0 + 64] = 0
    assert (out.astype(object) == want).all()
    Cp = np.zeros((sp, m, n), dtype=np.int8)
    Cp = oracle.gemm_rns_tiled(oracle.pack_u64(A, sp), oracle.pack_u64(B, sp), Cp, oentries)
    got = Cm.read_residues(sp)
    for e in oentries:  # planes each tile computes (the rest were never written: zero here)
        sl = (slice(0, e.selected_prefix), slice(e.row_offset, e.row_offset + e.row_extent),
              slice(e.col_offset, e.col_offset + e.col_extent))
        np.testing.assert_array_equal(got[sl], Cp[sl])
