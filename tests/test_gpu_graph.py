"""A resident step captured into a HIP graph and replayed.

The device entry points (rns8_mi355x_pack_*_device, _gemm_*_async,
_export_*_device) enqueue kernels only (no allocation, copy, memset or
synchronization for bounded and finite plans), so a caller can capture pack
-> GEMM -> export once and replay it. Every replay runs on new inputs written
into the same device buffers between replays (with eager library work and
synchronizations in between), and each replay's output is checked against the
exact product and against an eager run.
"""
import ctypes

import numpy as np
import pytest

import rns8_amd as r
from rns8_amd import hip, inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,n,k,bits", [(256, 256, 256, 20), (130, 70, 300, 18), (128, 128, 16384, 12)])
def test_captured_step_replays(gpu_ctx, m, n, k, bits):
    L = r.lib()
    bound = k << (2 * bits)
    desc = r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, m, n, k, bound=bound)
    plan = r.Plan(gpu_ctx, desc)
    P = plan.prefix
    mk = lambda rows, cols: r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, P))
    Am, Bm, Cm = mk(m, k), mk(k, n), mk(m, n)
    ws = r.Workspace(gpu_ctx, plan)
    dA, dB, dC, dS = hip.malloc(m * k * 8), hip.malloc(k * n * 8), hip.malloc(m * n * 8), hip.malloc(64)
    stream = hip.stream_create()
    vp = ctypes.c_void_p

    def step():
        r.check(L.rns8_mi355x_pack_i64_device(gpu_ctx.ptr, Am.ptr, vp(dA), k, 0, vp(stream)), "pack A")
        r.check(L.rns8_mi355x_pack_i64_device(gpu_ctx.ptr, Bm.ptr, vp(dB), n, 0, vp(stream)), "pack B")
        r.check(L.rns8_mi355x_gemm_rns_async(gpu_ctx.ptr, plan.ptr, Am.ptr, Bm.ptr, Cm.ptr, ws.ptr, vp(stream)),
                "gemm")
        r.check(L.rns8_mi355x_export_i64_device(gpu_ctx.ptr, plan.ptr, Cm.ptr, vp(dC), n, vp(dS), vp(stream)),
                "export")

    try:
        hip.capture_begin(stream)
        step()
        graph, exe = hip.capture_end(stream)
        try:
            for replay in range(3):
                A = inputs.int_range(inputs.operand_seed(700 + replay, "A"), (m, k), bits)
                B = inputs.int_range(inputs.operand_seed(700 + replay, "B"), (k, n), bits)
                hip.to_device(dA, A)
                hip.to_device(dB, B)
                hip.memset(dS, 0, 64)
                hip.memset(dC, 0, m * n * 8)
                hip.synchronize()
                hip.graph_launch(exe, stream)
                hip.stream_synchronize(stream)
                got = np.empty((m, n), dtype=np.int64)
                hip.from_device(got, dC)
                status = np.zeros(1, dtype=np.uint32)
                hip.from_device(status, dS)
                assert status[0] == 0
                np.testing.assert_array_equal(got, A @ B)
                # the same step run eagerly gives the same bytes
                hip.memset(dC, 0, m * n * 8)
                step()
                hip.stream_synchronize(stream)
                eager = np.empty((m, n), dtype=np.int64)
                hip.from_device(eager, dC)
                np.testing.assert_array_equal(eager, got)
        finally:
            hip.graph_destroy(graph, exe)
    finally:
        hip.stream_destroy(stream)
        for p in (dA, dB, dC, dS):
            hip.free(p)
