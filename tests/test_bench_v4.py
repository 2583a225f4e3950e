"""rns8-bench schema-v4 capture records (rns8_amd/bench_v4.py), without a device.

Pinned by the reference's own v4 fixtures (tests/golden/benchmark_schema/,
copied from tests/fixtures/benchmark_schema): a record built here has the
fixture's top-level and nested keys with the same JSON kinds, and the summary
statistics recomputed from each fixture's raw timings equal the summaries the
fixture stores (tools/benchmark_schema/core_shared.py:319-332 defines them).
"""
import json
from pathlib import Path

import numpy as np
import pytest

from rns8_amd import bench_v4

GOLDEN = Path(__file__).parent / "golden" / "benchmark_schema"
GLOBAL = json.loads((GOLDEN / "v4_bounded_i64_ck.json").read_text())
PER_TILE = json.loads((GOLDEN / "v4_bounded_i64_adaptive_hip.json").read_text())


def _kind(v):
    if v is None:
        return None
    if isinstance(v, bool):
        return "bool"
    if isinstance(v, (int, float)):
        return "number"
    return type(v).__name__


def _synthetic(per_tile):
    repeats = 3
    raw = {"planning": [1200], "scheduling": [4], "matrix_alloc": [300], "pack": [50, 60, 55],
           "rns_gemm": [90, 80, 85], "crt_export": [40, 41, 39], "end_to_end": [180, 181, 179]}
    if per_tile:
        raw["tile_bound_scan"] = [7]
    schedule = dict(PER_TILE["schedule_metadata"] if per_tile else GLOBAL["schedule_metadata"])
    backend = dict(PER_TILE["backend_metadata"])
    return bench_v4.build_record(
        semantics="bounded_i64", bound_kind="per_tile_max_abs" if per_tile else "global_max_abs",
        bound_mode="per_tile" if per_tile else "global", bound=0 if per_tile else 1 << 40, m=65, n=65, k=64,
        prefix=9, tile_m=64, tile_n=64, k_block_size=64, tile_bounds=[6, 2000, 3000000, 10 ** 9] if per_tile else None,
        schedule=schedule, backend=backend, seed=7, warmups=1, repeats=repeats, input_distribution="x",
        command_line="bench.py", device=dict(GLOBAL["device"]), raw=raw, checksum=123)


@pytest.mark.parametrize("per_tile", [False, True])
def test_record_has_the_fixture_layout(per_tile):
    rec = _synthetic(per_tile)
    ref = PER_TILE if per_tile else GLOBAL
    assert list(rec.keys()) == list(ref.keys())
    for key, want in ref.items():
        if want is not None and rec[key] is not None and key not in ("gpu_event_timings_us",
                                                                       "gpu_event_timing_summary_us"):
            assert _kind(rec[key]) == _kind(want), key
    for nested in ("backend_metadata", "schedule_metadata", "device", "hip_toolchain", "compiler",
                   "comparison_baseline"):
        assert set(rec[nested]) == set(ref[nested]), nested
    assert set(rec["backend_metadata"]["accumulator_safety"]) == set(ref["backend_metadata"]["accumulator_safety"])
    assert set(rec["timing_metadata"]) == set(ref["timing_metadata"])
    assert rec["timing_metadata"]["phase_order"] == ref["timing_metadata"]["phase_order"]
    assert set(rec["raw_timings_us"]) == set(ref["raw_timings_us"])
    if per_tile:
        assert set(rec["tile_bounds_u64"]) == set(ref["tile_bounds_u64"])
    # GPU event fields are null together when no events are collected
    assert rec["timing_metadata"]["gpu_event_timing"] is False
    assert rec["gpu_event_timings_us"] is None and rec["gpu_event_timing_summary_us"] is None
    assert rec["timing_metadata"]["gpu_event_phase_order"] is None


@pytest.mark.parametrize("ref", [GLOBAL, PER_TILE], ids=["global", "per_tile"])
def test_summaries_match_the_fixtures_own(ref):
    for phase, values in ref["raw_timings_us"].items():
        got = bench_v4.summary([float(v) for v in values])
        for key in ("avg", "median", "p95"):
            assert got[key] == pytest.approx(ref["timing_summary_us"][phase][key], rel=1e-5, abs=1e-2), (phase, key)


@pytest.mark.parametrize("per_tile", [False, True])
def test_record_averages_follow_raw(per_tile):
    rec = _synthetic(per_tile)
    raw = rec["raw_timings_us"]
    for field, phase in [("avg_planning_us", "planning"), ("avg_scheduling_us", "scheduling"),
                         ("avg_matrix_alloc_us", "matrix_alloc"), ("avg_pack_us", "pack"),
                         ("avg_rns_gemm_us", "rns_gemm"), ("avg_crt_export_us", "crt_export"),
                         ("avg_end_to_end_us", "end_to_end")]:
        assert rec[field] == pytest.approx(np.mean(raw[phase]))
    assert rec["schedule_query_us"] == pytest.approx(np.mean(raw["scheduling"]))
    for phase in ("pack", "rns_gemm", "crt_export", "end_to_end"):
        assert len(raw[phase]) == rec["repeats"]
    if per_tile:
        assert rec["tile_bound_scan_us"] == raw["tile_bound_scan"][0]


def test_checksum_is_word_fnv1a():
    # an independent fold in numpy's wrapping uint64 arithmetic
    rng = np.random.default_rng(0)
    words = rng.integers(0, 2 ** 63, size=(7, 5), dtype=np.int64)
    h = np.uint64(bench_v4.FNV_OFFSET)
    with np.errstate(over="ignore"):
        for w in words.reshape(-1).view(np.uint64):
            h = (h ^ w) * np.uint64(bench_v4.FNV_PRIME)
    assert bench_v4.checksum_u64(words) == int(h)
    assert bench_v4.checksum_u64(np.zeros((0,), dtype=np.uint64)) == bench_v4.FNV_OFFSET


def test_phase_count_is_enforced():
    with pytest.raises(ValueError):
        raw = {"planning": [1], "scheduling": [1], "matrix_alloc": [1], "pack": [1], "rns_gemm": [1],
               "crt_export": [1], "end_to_end": [1]}
        bench_v4.build_record(semantics="bounded_i64", bound_kind="global_max_abs", bound_mode="global", bound=1,
                              m=1, n=1, k=1, prefix=1, tile_m=128, tile_n=128, k_block_size=1, tile_bounds=None,
                              schedule={}, backend={"selected_kernel": "x"}, seed=0, warmups=0, repeats=2,
                              input_distribution="", command_line="", device={}, raw=raw, checksum=0)
