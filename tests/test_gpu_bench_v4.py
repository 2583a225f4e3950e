"""The schema-v4 capture lane on the GPU: the record of a real run has the
reference fixtures' layout, and its checksum is the checksum of the exact
product (so the exported values it summarizes are the right ones)."""
import numpy as np
import pytest

from rns8_amd import bench_v4, inputs
from test_bench_v4 import GLOBAL, PER_TILE

pytestmark = pytest.mark.gpu


def _layout(rec, ref):
    assert list(rec.keys()) == list(ref.keys())
    for nested in ("backend_metadata", "schedule_metadata", "device", "timing_metadata"):
        assert set(rec[nested]) == set(ref[nested]), nested


def test_global_capture(gpu_ctx):
    m, n, k = 96, 130, 200
    A = inputs.int_range(inputs.operand_seed(3, "A"), (m, k), 20)
    B = inputs.int_range(inputs.operand_seed(3, "B"), (k, n), 20)
    rec, C = bench_v4.capture_bounded(gpu_ctx, A, B, signed=True, bound=1 << 62, budget=9, forced=True,
                                      warmups=1, repeats=3, seed=3, input_distribution="splitmix64_test")
    _layout(rec, GLOBAL)
    exact = A @ B
    np.testing.assert_array_equal(C, exact)
    assert rec["checksum_u64"] == bench_v4.checksum_u64(exact)
    assert rec["prefix"] == 9 and rec["repeats"] == 3 and len(rec["raw_timings_us"]["rns_gemm"]) == 3
    assert rec["backend_metadata"]["selected_kernel"] == rec["selected_kernel"]


def test_per_tile_capture(gpu_ctx):
    m, n, k = 200, 130, 50
    A = inputs.int_range(inputs.operand_seed(4, "A"), (m, k), 20)
    A[:128] >>= 15
    B = inputs.uint_range(inputs.operand_seed(4, "B"), (k, n), 20).astype(np.int64)
    bounds = lambda: [k << (25 if t < 2 else 40) for t in range(4)]
    rec, C = bench_v4.capture_bounded(gpu_ctx, A, B, signed=True, budget=9, tile_bounds_fn=bounds, tile=128,
                                      warmups=0, repeats=2, seed=4)
    _layout(rec, PER_TILE)
    np.testing.assert_array_equal(C, A @ B)
    assert rec["schedule_metadata"]["prefix_group_count"] == 2
    assert rec["tile_bounds_u64"]["count"] == 4
