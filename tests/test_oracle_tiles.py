"""Per-tile bounded schedules in the CPU oracle.

The schedule restatement (api_plan_schedule.inc:109-261) is pinned by the
reference's own unit-test expectations (tests/golden/reference_tile_kats.json,
transcribed from test_bounded_gemm_schedule_cases.inc and
test_bounded_gemm_per_tile_cases.inc). The tiled GEMM and export
(cpu_reference.cpp:231-257, api_export.cpp:365-410) are pinned by those
oneshot KATs and by exact integer products: random per-tile bounds set from
the true per-tile maxima, every exported value equal to the Python big-int
product, planes above a tile's prefix untouched, and a bound one below a
tile's maximum rejected.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle

KATS = json.loads((Path(__file__).parent / "golden" / "reference_tile_kats.json").read_text())
SENTINEL = -91


def _mask(n, set_indices):
    m = np.zeros(n, dtype=np.uint8)
    m[list(set_indices)] = 1
    return m


@pytest.mark.parametrize("case", KATS["schedules"], ids=lambda c: c["name"])
def test_schedule_matches_reference_expectations(case):
    za = zb = None
    if "zero_a_rows_set" in case:
        za = _mask(case["m"], case["zero_a_rows_set"])
        zb = _mask(case["n"], case["zero_b_cols_set"])
    st, entries, summary = oracle.tile_schedule(case["signed"], case["m"], case["n"], case["tile_m"], case["tile_n"],
                                                case["bounds"], case["budget"], case["flags"], za, zb)
    assert st == 0
    for key, want in case["summary"].items():
        assert getattr(summary, key) == want, key
    for idx, fields in case["entries"].items():
        for key, want in fields.items():
            assert getattr(entries[int(idx)], key) == want, (idx, key)


def test_schedule_rejections():
    # I64 bound above 2^63 is invalid; a bound needing more than the budget is a range error
    assert oracle.tile_schedule(True, 65, 65, 64, 64, [1 << 63, 1, 1, (1 << 63) + 1], 9)[0] == 1
    assert oracle.tile_schedule(False, 65, 65, 64, 64, [1, 1, 1, 1 << 40], 4)[0] == 5
    assert oracle.tile_schedule(False, 65, 65, 64, 64, [1, 1, 1], 9)[0] == 1  # wrong bound count


def _oneshot(signed, A, B, tile, bounds, flags, budget=9):
    m, n = A.shape[0], B.shape[1]
    st, entries, summary = oracle.tile_schedule(signed, m, n, tile, tile, bounds, budget, flags)
    assert st == 0
    storage = summary.max_selected
    pack = oracle.pack_i64 if signed else oracle.pack_u64
    Ap, Bp = pack(A, storage), pack(B, storage)
    Cp = np.full((storage, m, n), SENTINEL, dtype=np.int8)
    Cp = oracle.gemm_rns_tiled(Ap, Bp, Cp, entries)
    return oracle.export_tiled(Cp, tile, tile, entries, bounds, signed), entries, Cp


@pytest.mark.parametrize("case", KATS["oneshots"], ids=lambda c: c["name"])
def test_oneshot_kats(case):
    m, n, k = case["m"], case["n"], case["k"]
    dt = np.int64 if case["signed"] else np.uint64
    a, b = case["a_col"], case["b_row"]
    A = np.array([[a["lo"] if r < a["split"] else a["hi"]] for r in range(m)], dtype=dt)
    B = np.array([[b["lo"] if c < b["split"] else b["hi"] for c in range(n)]], dtype=dt)
    (st, out), _, _ = _oneshot(case["signed"], A, B, case["tile"], case["bounds"], case["flags"])
    assert st == case["status"]
    if st == 0:
        want = np.array([[int(A[r, 0]) * int(B[0, c]) for c in range(n)] for r in range(m)], dtype=object)
        assert (out.astype(object) == want).all()
    else:
        assert not out.any()  # dst untouched (zero-initialized here)


@pytest.mark.parametrize("seed", range(6))
def test_random_tiles_exact_products(seed):
    rng = np.random.default_rng(seed)
    signed = bool(seed % 2)
    tile = [64, 128][seed % 2 == 0]
    m, n, k = int(rng.integers(1, 300)), int(rng.integers(1, 300)), int(rng.integers(1, 40))
    dt = np.int64 if signed else np.uint64
    # per-row / per-column magnitudes so tiles need very different prefixes
    row_bits = rng.integers(1, 28, size=m)
    col_bits = rng.integers(1, 28, size=k)
    A = np.array([[int(rng.integers(0, 1 << int(row_bits[r]))) * (-1 if signed and rng.random() < 0.5 else 1)
                   for _ in range(k)] for r in range(m)], dtype=dt)
    B = np.array([[int(rng.integers(0, 1 << int(col_bits[j]))) for _ in range(n)] for j in range(k)], dtype=dt)
    exact = A.astype(object) @ B.astype(object)
    tr, tc = -(-m // tile), -(-n // tile)
    bounds = []
    for t in range(tr * tc):
        r0, c0 = (t // tc) * tile, (t % tc) * tile
        blk = exact[r0:r0 + tile, c0:c0 + tile]
        bounds.append(int(max(abs(int(x)) for x in blk.flat)))
    (st, out), entries, Cp = _oneshot(signed, A, B, tile, bounds, 0)
    assert st == 0
    assert (out.astype(object) == exact).all()
    # planes at or above a tile's selected prefix were never written
    for e in entries:
        blk = Cp[e.selected_prefix:, e.row_offset:e.row_offset + e.row_extent, e.col_offset:e.col_offset + e.col_extent]
        assert (blk == SENTINEL).all()
    # one tile's bound one below its true maximum is a range error
    hot = int(np.argmax(bounds))
    if bounds[hot] > 0:
        low = list(bounds)
        low[hot] -= 1
        (st2, _), _, _ = _oneshot(signed, A, B, tile, low, 0)
        assert st2 == 5
