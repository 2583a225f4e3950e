"""Plan schedules through the C ABI, without a device.

`rns8_mi355x_plan_schedule` reports what rns8_get_plan_schedule_info and
rns8_get_plan_tile_schedule return for the plan a descriptor creates. It is
checked against the reference's own unit-test expectations
(tests/golden/reference_tile_kats.json) and, field by field, against the
oracle's restatement of api_plan_schedule.inc for random per-tile
descriptors, including rejections.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
import rns8_amd as r

KATS = json.loads((Path(__file__).parent / "golden" / "reference_tile_kats.json").read_text())
ENTRY_FIELDS = ["flags", "tile_row", "tile_col", "row_offset", "col_offset", "row_extent", "col_extent",
                "required_prefix", "selected_prefix", "group_index", "range_bit_length"]
INFO_FROM_ORACLE = {"tile_rows": "tile_rows", "tile_cols": "tile_cols", "tile_count": "tile_count",
                    "min_required_prefix": "min_required", "max_required_prefix": "max_required",
                    "min_selected_prefix": "min_selected", "max_selected_prefix": "max_selected",
                    "prefix_group_count": "group_count", "adaptive_prefix_active": "adaptive_prefix",
                    "adaptive_skip_active": "adaptive_skip", "range_bit_length": "range_bits", "flags": "flags",
                    "zero_a_row_count": "zero_a_row_count", "zero_b_col_count": "zero_b_col_count",
                    "zero_row_col_product_count": "zero_row_col_product_count"}
KAT_TO_INFO = {v: k for k, v in INFO_FROM_ORACLE.items()}


def _mask(n, set_indices):
    m = np.zeros(n, dtype=np.uint8)
    m[list(set_indices)] = 1
    return m


def _desc(signed, m, n, k, tile_m, tile_n, bounds, budget, flags, za=None, zb=None):
    sem = r.BOUNDED_I64 if signed else r.BOUNDED_U64
    bk = r.abi.BOUND_PER_TILE_MAX_ABS if signed else r.abi.BOUND_PER_TILE_MAX_UNSIGNED
    return r.gemm_desc(sem, bk, m, n, k, max_prefix=budget, flags=flags, tile_m=tile_m, tile_n=tile_n,
                       tile_bounds=bounds, zero_a_rows=za, zero_b_cols=zb)


@pytest.mark.parametrize("case", KATS["schedules"], ids=lambda c: c["name"])
def test_reference_schedule_expectations(case):
    za = zb = None
    if "zero_a_rows_set" in case:
        za = _mask(case["m"], case["zero_a_rows_set"])
        zb = _mask(case["n"], case["zero_b_cols_set"])
    d = _desc(case["signed"], case["m"], case["n"], 7, case["tile_m"], case["tile_n"], case["bounds"], case["budget"],
              case["flags"], za, zb)
    st, info, entries = r.plan_schedule(d)
    assert st == r.SUCCESS
    assert info.bound_contract == b"per_tile_output_bounds"
    for key, want in case["summary"].items():
        if key == "collapsed":
            continue
        assert getattr(info, KAT_TO_INFO[key]) == want, key
    for idx, fields in case["entries"].items():
        for key, want in fields.items():
            assert getattr(entries[int(idx)], key) == want, (idx, key)


def test_global_schedule_grid():
    # reference test_bounded_gemm_schedule_cases.inc:69-124
    d = r.gemm_desc(r.BOUNDED_U64, r.abi.BOUND_GLOBAL_MAX_UNSIGNED, 130, 129, 7, bound=1000, tile_m=64, tile_n=64)
    st, info, entries = r.plan_schedule(d)
    assert st == r.SUCCESS
    assert (info.tile_rows, info.tile_cols, info.tile_count) == (3, 3, 9)
    assert (info.min_required_prefix, info.max_required_prefix) == (2, 2)
    assert (info.min_selected_prefix, info.max_selected_prefix) == (2, 2)
    assert (info.prefix_group_count, info.adaptive_prefix_active, info.adaptive_skip_active) == (1, 0, 1)
    assert info.range_bit_length == 10
    assert info.bound_contract == b"global_output_bound"
    f, b = entries[0], entries[-1]
    assert (f.row_extent, f.col_extent, f.required_prefix, f.selected_prefix, f.range_bit_length) == (64, 64, 2, 2, 10)
    assert (b.tile_row, b.tile_col, b.row_offset, b.col_offset, b.row_extent, b.col_extent) == (2, 2, 128, 128, 2, 1)


@pytest.mark.parametrize("seed", range(40))
def test_random_descriptors_match_oracle(seed):
    rng = np.random.default_rng(1000 + seed)
    signed = bool(rng.integers(0, 2))
    m, n = int(rng.integers(1, 700)), int(rng.integers(1, 700))
    tile_m, tile_n = [0, 64, 128, 256, 512][rng.integers(0, 5)], [0, 64, 128, 256, 512][rng.integers(0, 5)]
    tm, tn = tile_m or 128, tile_n or 128
    count = -(-m // tm) * -(-n // tn)
    budget = int(rng.integers(1, 10))
    flags = int(rng.choice([0, 1, 2, 4, 6, 7]))
    top = 63 if signed else 64
    bits = rng.integers(0, top + 1, size=count)
    bounds = [0 if b == 0 else int(rng.integers(1 << (int(b) - 1), (1 << int(b)) - 1, endpoint=True, dtype=np.uint64))
              for b in bits]
    za = zb = None
    if flags & 4:
        za = (rng.random(m) < 0.02).astype(np.uint8)
        zb = (rng.random(n) < 0.02).astype(np.uint8)
    d = _desc(signed, m, n, 5, tile_m, tile_n, bounds, budget, flags, za, zb)
    st, info, entries = r.plan_schedule(d)
    ost, oentries, osum = oracle.tile_schedule(signed, m, n, tile_m, tile_n, bounds, budget, flags, za, zb)
    assert st == ost
    if st != r.SUCCESS:
        return
    for ifield, ofield in INFO_FROM_ORACLE.items():
        assert getattr(info, ifield) == getattr(osum, ofield), ifield
    assert len(entries) == len(oentries) == count
    for e, o in zip(entries, oentries):
        for f in ENTRY_FIELDS:
            assert getattr(e, f) == getattr(o, f), f


def test_per_tile_rejections():
    # wrong bound count, I64 bound above 2^63, bound beyond the budget, stray flags on global plans
    assert r.plan_schedule(_desc(False, 65, 65, 1, 64, 64, [1, 1, 1], 9, 0))[0] == r.INVALID_ARGUMENT
    assert r.plan_schedule(_desc(True, 65, 65, 1, 64, 64, [1, 1, 1, (1 << 63) + 1], 9, 0))[0] == r.INVALID_ARGUMENT
    assert r.plan_schedule(_desc(False, 65, 65, 1, 64, 64, [1, 1, 1, 1 << 40], 4, 0))[0] == r.RANGE_ERROR
    g = r.gemm_desc(r.BOUNDED_U64, r.abi.BOUND_GLOBAL_MAX_UNSIGNED, 1, 1, 1, bound=1,
                    flags=r.abi.PLAN_ALLOW_PROVEN_ZERO_TILE_SKIPS)
    assert r.plan_schedule(g)[0] == r.INVALID_ARGUMENT
    # masks without the opt-in flag, and a mask value other than 0/1
    za, zb = _mask(65, [0]), _mask(65, [64])
    assert r.plan_schedule(_desc(False, 65, 65, 1, 64, 64, [9] * 4, 9, 0, za, zb))[0] == r.INVALID_ARGUMENT
    za[1] = 2
    assert r.plan_schedule(_desc(False, 65, 65, 1, 64, 64, [9] * 4, 9, 4, za, zb))[0] == r.INVALID_ARGUMENT
