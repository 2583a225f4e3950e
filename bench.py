#!/usr/bin/env python3
"""Benchmark: exact int64 GEMM effective TOPS at 4096^3, prefix 9, on one MI355X.

Workload: RNS8_BOUNDED_I64, M = N = K = 4096, A and
B int64 uniform in [-2^25, 2^25) from SplitMix64 streams, declared bound 2^62
with FORCE_FIXED_PREFIX and max_prefix 9 (moduli 256 ... 227). One step =
pack A + pack B (device int64 -> residue planes) + 9-plane int8 MFMA GEMM +
Garner reconstruct to device int64, all through the rns8 C ABI device-resident
entry points on one HIP stream. Inputs are resident in HBM before timing.

Printed JSON: value = 2*M*N*K / (ms_per_step) in TOPS (effective exact-integer
ops); roofline = the plane-GEMM kernel against the dense int8 MFMA peak
(2*M*N*K*P int8 ops per launch / average launch time, HIP events on the
launch stream); cpu_baseline = the CPU oracle (own restatement of the
reference CPU_REFERENCE path) on a bounded row sample of the same GEMM, whose
rows are also compared bit-exactly against the GPU output.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POPS
PEAK_HBM_GBS = 8000.0

CONFIGS = {
    # name: (semantics, m, n, k, input bits, bound, prefix budget, forced)
    "c3": ("i64", 4096, 4096, 4096, 25, 1 << 62, 9, True),
    "c1": ("i64", 256, 256, 256, 20, 256 << 40, 0, False),
    "c5": ("u64", 128, 128, 65536, 23, 1 << 62, 0, False),
    # per-tile bounds (128 x 128 tiles) on C3's shape: A's tile rows cycle
    # through magnitudes 2^1 .. 2^25, so tiles select prefixes 5 .. 9
    "tiled": ("i64", 4096, 4096, 4096, 25, 1 << 62, 9, False),
    # skinny products (the reference's GEMV lanes, N = 1 and N <= 8, and its
    # persistent-small kernel, M * N <= 64): the GEMM stage is bound by reading
    # A's planes once
    "gemv1": ("i64", 8192, 1, 8192, 25, 1 << 62, 9, True),
    "gemv8": ("i64", 8192, 8, 8192, 25, 1 << 62, 9, True),
    "small64": ("i64", 8, 8, 1 << 20, 25, 1 << 62, 9, True),
}
SKINNY = ("gemv1", "gemv8", "small64")
# configs whose default step is the fused native-input GEMM (--packed: packs + plane GEMM)
FUSED_DEFAULT = ("c5", "gemv1", "gemv8")
# grouped resident GEMM: GROUP_TASKS same-shape int64 tasks per step
GROUPED = ("i64", 1024, 1024, 1024, 25, 1 << 62, 9, True)
GROUP_TASKS = 8
TILED_EDGE = 128
TILED_ROW_BITS = [1, 5, 9, 13, 17, 21, 25]


class StageTimer:
    """HIP events at the stage boundaries of `steps` back-to-back steps on one
    stream. Nothing synchronizes between the steps, so each stage runs as it
    does in the timed pass; the elapsed times are read once, after the last
    step, and averaged per stage."""

    def __init__(self, steps: int, marks: int, stream):
        from rns8_amd import hip

        self.hip = hip
        self.ev = [[hip.event_create() for _ in range(marks)] for _ in range(steps)]
        self.stream = stream

    def marker(self, step: int):
        return lambda i: self.hip.event_record(self.ev[step][i], self.stream)

    def stage_ms(self) -> np.ndarray:
        self.hip.stream_synchronize(self.stream)
        t = [[self.hip.event_elapsed_ms(e[i], e[i + 1]) for i in range(len(e) - 1)] for e in self.ev]
        return np.array(t).mean(axis=0)

    def destroy(self) -> None:
        for row in self.ev:
            for e in row:
                self.hip.event_destroy(e)


def _no_mark(_i: int) -> None:
    pass


def settle(step, steps: int, sync) -> None:
    """Runs `steps` steps back to back before the warmup. After the GPU has
    idled (uploads, allocation), the power controller first lets the clock
    overshoot, then holds it down hard once the matrix cores load up, and
    climbs back to the sustained clock over ~25 C3 steps; a short warmup
    alone leaves the timed steps inside that transient."""
    for _ in range(steps):
        step()
    sync()


def attainable_mfma(achieved: float) -> dict:
    """The dense int8 MFMA rate this MI355X sustains with random operand bytes
    (the statistics of residue planes), measured after the timed region by
    rns8_amd/probe/librns8_probe.so: every CU issuing back-to-back
    v_mfma_i32_32x32x32_i8 from registers, ~50 ms so the power controller has
    settled. The chip is power-limited on such operands, so this, not the
    5.0 POP/s peak, is the ceiling a GEMM on this data can approach; zero
    operands are measured beside it for the clock contrast."""
    import ctypes as C

    lib = C.CDLL(str(ROOT / "rns8_amd" / "probe" / "librns8_probe.so"))
    fn = lib.rns8_probe_mfma_rate
    fn.restype = C.c_int
    fn.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_double)]
    out = {}
    for key, rnd in (("random", 1), ("zero", 0)):
        tops, ghz = C.c_double(), C.c_double()
        rc = fn(rnd, 2000, 10, 30, C.byref(tops), C.byref(ghz))
        if rc != 0:
            raise RuntimeError(f"rns8_probe_mfma_rate failed with HIP error {rc}")
        out[key] = (tops.value, ghz.value)
    rt, rg = out["random"]
    zt, zg = out["zero"]
    log(f"[bench] MFMA probe: random operands {rt:.0f} TOP/s at {rg:.3f} GHz, zero operands {zt:.0f} TOP/s at "
        f"{zg:.3f} GHz")
    return {"value": round(rt, 1), "unit": "TOP/s", "clock_ghz": round(rg, 3), "frac": round(achieved / rt, 4),
            "zero_operands": {"value": round(zt, 1), "clock_ghz": round(zg, 3)},
            "source": "rns8_amd/probe: back-to-back v_mfma_i32_32x32x32_i8 on every CU with random int8 "
                      "operands, measured after the timed region"}


def back_to_back_ms(call, stream: int, n: int) -> float:
    """Mean time of one `call` over n back-to-back calls on `stream` (HIP
    events around them all, after 3 untimed calls)."""
    from rns8_amd import hip

    for _ in range(3):
        call()
    hip.stream_synchronize(stream)
    e0, e1 = hip.event_create(), hip.event_create()
    hip.event_record(e0, stream)
    for _ in range(n):
        call()
    hip.event_record(e1, stream)
    hip.stream_synchronize(stream)
    ms = hip.event_elapsed_ms(e0, e1) / n
    hip.event_destroy(e0)
    hip.event_destroy(e1)
    return ms


def attainable_streams(stages: dict) -> dict:
    """For each memory-bound stage (name -> (bytes read, bytes written, ms
    per launch over back-to-back launches)), its algorithmic rate beside the
    rate a plain stream with the same reads and writes reaches on this
    MI355X, measured right after by rns8_amd/probe/librns8_probe.so (16-byte
    loads and stores, each wave instruction covering 1 KB; 20 back-to-back
    launches after 3 untimed ones, so both sides carry the same inter-launch
    gaps). Mixed read/write
    streams run well below the 8 TB/s peak, and below it the further the
    larger they are (the 256 MB Infinity Cache holds less of them), so this
    is the ceiling a pack or an export of that size can approach."""
    import ctypes as C

    lib = C.CDLL(str(ROOT / "rns8_amd" / "probe" / "librns8_probe.so"))
    fn = lib.rns8_probe_hbm_stream
    fn.restype = C.c_int
    fn.argtypes = [C.c_uint64, C.c_uint64, C.c_int, C.c_int, C.POINTER(C.c_double)]
    out = {}
    for name, (rd, wr, ms) in stages.items():
        gbps = C.c_double()
        rc = fn(rd // 16 * 16, wr // 16 * 16, 3, 20, C.byref(gbps))
        if rc != 0:
            raise RuntimeError(f"rns8_probe_hbm_stream failed with HIP error {rc}")
        achieved = (rd + wr) / (ms * 1e-3) / 1e9
        out[name] = {"read_bytes": rd, "write_bytes": wr, "ms": round(ms, 4), "achieved": round(achieved, 1),
                     "attainable": round(gbps.value, 1), "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "frac_of_attainable": round(achieved / gbps.value, 4)}
        log(f"[bench] stream probe {name}: {rd / 1e6:.1f} MB read + {wr / 1e6:.1f} MB written, stage "
            f"{1e3 * ms:.1f} us = {achieved:.0f} GB/s, plain stream {gbps.value:.0f} GB/s")
    out["source"] = ("rns8_amd/probe: a streaming kernel reading and writing the stage's algorithmic bytes; both "
                     "sides timed over back-to-back launches after the timed region")
    return out


def optional_probe(probe, *args):
    """A rate probe's report, or None when it fails: the probes give context
    beside the measured line and must not cost the line itself."""
    try:
        return probe(*args)
    except (OSError, RuntimeError) as err:
        log(f"[bench] probe {probe.__name__} failed, reported as null: {err}")
        return None


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--settle-steps", type=int, default=30,
                    help="steps run back to back before the warmup, so the timed steps do not start inside the "
                         "power controller's post-idle clock transient (reported as config.settle_steps; 0 disables)")
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS) + ["grouped", "c2", "c4"])
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU baseline sample time")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--packed", action="store_true",
                    help="c5/gemv1/gemv8: two packs and the plane GEMM in place of the fused native-input GEMM (the "
                         "default route for these shapes)")
    ap.add_argument("--fused", action="store_true",
                    help="c1/c3: one fused native-input GEMM (rns8_mi355x_gemm_native_*_async) in place of the two "
                         "packs and the plane GEMM")
    ap.add_argument("--host-pack", action="store_true",
                    help="time the exact-wide host-array packs (host range proof + upload + pack) and the GEMM's "
                         "admission at C4's operands instead")
    ap.add_argument("--oneshot", action="store_true",
                    help="time the host-buffer oneshot entry point instead (PCIe transfers included)")
    ap.add_argument("--graph", action="store_true",
                    help="capture one step into a HIP graph and time graph replays in the back-to-back pass")
    ap.add_argument("--rns8-bench-json", default="", metavar="PATH",
                    help="also run the host-API lane on the same inputs and write an rns8-bench schema-v4 capture")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a device copy of BYTES (counter calibration) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration, max(args.steps, 1))
    if args.oneshot:
        return oneshot_rate(args)
    if args.host_pack:
        return host_pack_rate(args)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported in this build "
              "(across GPUs the path would shard by output row blocks, one share of rows per GPU)", file=sys.stderr)
        return 2
    if args.config == "grouped":
        return grouped_bench(args)
    if args.config in ("c2", "c4"):
        return finite_or_wide_bench(args)

    import rns8_amd as r
    from rns8_amd import hip, inputs

    sem, M, N, K, bits, bound, budget, forced = CONFIGS[args.config]
    signed = sem == "i64"
    dt = np.int64 if signed else np.uint64
    log(f"[bench] config {args.config}: {sem} {M}x{N}x{K} bits={bits}")
    if signed:
        A = inputs.int_range(inputs.operand_seed(args.seed, "A"), (M, K), bits)
        B = inputs.int_range(inputs.operand_seed(args.seed, "B"), (K, N), bits)
    else:
        A = inputs.uint_range(inputs.operand_seed(args.seed, "A"), (M, K), bits)
        B = inputs.uint_range(inputs.operand_seed(args.seed, "B"), (K, N), bits)

    tiled = args.config == "tiled"
    ctx = r.Context()
    semantics = r.BOUNDED_I64 if signed else r.BOUNDED_U64
    bk = r.BOUND_GLOBAL_MAX_ABS if signed else r.BOUND_GLOBAL_MAX_UNSIGNED
    tile = 0
    if tiled:
        A, tile_bounds = tiled_operands(A, bits, N, K)
        bk, tile = r.BOUND_PER_TILE_MAX_ABS, TILED_EDGE
        desc = r.gemm_desc(semantics, bk, M, N, K, max_prefix=budget, tile_m=tile, tile_n=tile,
                           tile_bounds=tile_bounds)
    else:
        desc = r.gemm_desc(semantics, bk, M, N, K, bound=bound, max_prefix=budget,
                           flags=r.PLAN_FORCE_FIXED_PREFIX if forced else 0)
    plan = r.Plan(ctx, desc)
    P = plan.prefix
    Am = r.Matrix(ctx, r.matrix_desc(M, K, semantics, bk, P, tile_m=tile, tile_n=tile))
    Bm = r.Matrix(ctx, r.matrix_desc(K, N, semantics, bk, P, tile_m=tile, tile_n=tile))
    Cm = r.Matrix(ctx, r.matrix_desc(M, N, semantics, bk, P, tile_m=tile, tile_n=tile))
    ws = r.Workspace(ctx, plan)
    # int8 MFMA ops the GEMM must do: every plane of every cell, or, per tile,
    # the planes its schedule selects
    gemm_ops = 2.0 * M * N * K * P
    if tiled:
        gemm_ops = sum(2.0 * e.row_extent * e.col_extent * K * e.selected_prefix for e in plan.tile_schedule())
    log(f"[bench] prefix {P}")

    dA = hip.malloc(A.nbytes)
    dB = hip.malloc(B.nbytes)
    dC = hip.malloc(M * N * 8)
    dS = hip.malloc(64)
    hip.to_device(dA, A)
    hip.to_device(dB, B)
    hip.memset(dS, 0, 64)
    stream = hip.stream_create()
    L = r.lib()
    pack = L.rns8_mi355x_pack_i64_device if signed else L.rns8_mi355x_pack_u64_device
    export = L.rns8_mi355x_export_i64_device if signed else L.rns8_mi355x_export_u64_device
    native = L.rns8_mi355x_gemm_native_i64_async if signed else L.rns8_mi355x_gemm_native_u64_async
    # tall-skinny C5 and the GEMVs run the fused native-input GEMM unless --packed asks for
    # the two packs and the split-K plane GEMM
    fused = args.fused or (args.config in FUSED_DEFAULT and not args.packed)
    if fused and tiled:
        log("[bench] --fused applies to plans with a global bound only")
        return 2

    def step(mark=_no_mark):
        mark(0)
        if fused:
            # the packs are inside the fused launch: their stages are empty
            mark(1)
            mark(2)
            r.check(native(ctx.ptr, plan.ptr, dA, K, dB, N, Cm.ptr, ws.ptr, stream), "fused gemm")
        else:
            r.check(pack(ctx.ptr, Am.ptr, dA, K, 0, stream), "pack A")
            mark(1)
            r.check(pack(ctx.ptr, Bm.ptr, dB, N, 0, stream), "pack B")
            mark(2)
            r.check(L.rns8_mi355x_gemm_rns_async(ctx.ptr, plan.ptr, Am.ptr, Bm.ptr, Cm.ptr, ws.ptr, stream), "gemm")
        mark(3)
        r.check(export(ctx.ptr, plan.ptr, Cm.ptr, dC, N, dS, stream), "export")
        mark(4)

    settle(step, args.settle_steps, lambda: hip.stream_synchronize(stream))
    for _ in range(args.warmup):
        step()
    hip.stream_synchronize(stream)
    log(f"[bench] {args.settle_steps} settle steps and {args.warmup} warmup steps done")

    # end-to-end pass: K steps back to back, bracketed by synchronization
    graph = None
    if args.graph:
        # the device entry points only enqueue kernels, so one step captures
        hip.capture_begin(stream)
        step()
        graph = hip.capture_end(stream)
        hip.graph_launch(graph[1], stream)
        hip.stream_synchronize(stream)
    hip.synchronize()
    start, stop = hip.event_create(), hip.event_create()
    t0 = time.perf_counter()
    hip.event_record(start, stream)
    for s in range(args.steps):
        if graph:
            hip.graph_launch(graph[1], stream)
        else:
            step()
    hip.event_record(stop, stream)
    hip.stream_synchronize(stream)
    t1 = time.perf_counter()
    hip.synchronize()
    ms_total = hip.event_elapsed_ms(start, stop)
    ms_per_step = ms_total / args.steps
    log(f"[bench] {args.steps} steps: {ms_total:.3f} ms (host clock {1e3 * (t1 - t0):.3f} ms)")

    # stage timing pass, after the timed one: K more steps back to back with
    # events between the stages
    timer = StageTimer(args.steps, 5, stream)
    for s in range(args.steps):
        step(timer.marker(s))
    stage = timer.stage_ms()
    timer.destroy()
    log(f"[bench] stage ms: packA {stage[0]:.4f} packB {stage[1]:.4f} gemm {stage[2]:.4f} export {stage[3]:.4f}")

    status = np.zeros(16, dtype=np.uint32)
    hip.from_device(status, dS)
    Cout = np.empty((M, N), dtype=dt)
    hip.from_device(Cout, dC)
    ops = 2.0 * M * N * K
    value = ops / (ms_per_step * 1e-3) / 1e12
    achieved = gemm_ops / (stage[2] * 1e-3) / 1e12
    if tiled:
        workload = (f"RNS8_BOUNDED_I64 {M}x{N}x{K}, per-tile bounds ({tile}x{tile} tiles, A tile rows at "
                    f"2^{TILED_ROW_BITS} cycling, B at 2^{bits}), storage prefix {P}, pack+GEMM+Garner device-resident")
        kernel = "plane_gemm_kernel<Cfg<4,4>,1,true,true,false> (listed 256x256 units, persistent)"
    elif args.config == "c3":
        workload = f"RNS8_BOUNDED_I64 {M}x{N}x{K} prefix {P} (FORCE_FIXED_PREFIX), pack+GEMM+Garner device-resident"
        kernel = "plane_gemm_kernel<Cfg<4,4>,1,true,false,false> (256x256 tiles, persistent)"
    elif args.config == "c5":
        workload = f"c5 {sem} {M}x{N}x{K} prefix {P}, pack+GEMM+Garner device-resident"
        kernel = "plane_gemm_kernel<Cfg<2,2>,2,true,false,false> K split + residue_finalize_kernel"
    else:
        workload = f"{args.config} {sem} {M}x{N}x{K} prefix {P}, pack+GEMM+Garner device-resident"
        kernel = "plane_gemm_kernel<Cfg<2,2>,2,true,false,false> (128x128 tiles, persistent)"

    if args.config == "c3":
        metric = "exact int64 GEMM effective TOPS (2MNK/s) at 4096\u00b3 prefix 9; % int8 MFMA peak"
    else:
        metric = f"exact {'int64' if signed else 'uint64'} GEMM effective TOPS (2MNK/s) at {M}x{N}x{K} prefix {P}"
    roofline = {
        "bound": "mfma", "kernel": kernel, "achieved": round(achieved, 2), "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
        "frac": round(achieved / PEAK_INT8_TOPS, 4), "per_launch_ops": gemm_ops,
    }
    traffic_kernels, traffic_workload = ["plane_gemm_kernel"], args.config
    if fused:
        # pack and GEMM in one pass: the native operands are read (8 bytes per
        # element) and the C planes written; HBM bounds it for tall-skinny shapes
        # results at most 16 columns wide take the skinny form (B's planes
        # first, then A converted in registers) while its workspace fits 256 MiB
        skinny_form = N <= 16 and P * 16 * ((K + 63) // 64 * 64) <= (256 << 20)
        kernel = ("pack_bt_kernel + fused_skinny_kernel<Signed,G,First256> + residue_finalize_kernel" if skinny_form
                  else "fused_native_kernel<Signed,NP> + residue_finalize_kernel")
        workload = workload.replace("pack+GEMM", "fused pack+GEMM")
        gemm_bytes = 8 * K * (M + N) + P * M * N
        gbs = gemm_bytes / ((stage[0] + stage[1] + stage[2]) * 1e-3) / 1e9
        roofline = {"bound": "hbm", "kernel": kernel, "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(gbs / PEAK_HBM_GBS, 4), "per_launch_bytes": gemm_bytes}
        traffic_kernels = (["pack_bt_kernel", "fused_skinny_kernel", "residue_finalize_kernel"] if skinny_form
                           else ["fused_native_kernel", "residue_finalize_kernel"])
    elif args.config in SKINNY:
        # at most 16 columns: the GEMM reads A's planes once and B's (padded
        # to 16 columns) once, so HBM bounds it
        kernel = plan.selected_kernel()
        gemm_bytes = P * (M * K + K * 16 + M * 16)
        gbs = gemm_bytes / (stage[2] * 1e-3) / 1e9
        roofline = {"bound": "hbm", "kernel": kernel, "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(gbs / PEAK_HBM_GBS, 4), "per_launch_bytes": gemm_bytes}
        traffic_kernels = ["skinny_gemm_kernel"] + (["residue_finalize_kernel"] if "K split" in kernel else [])
        if args.config in FUSED_DEFAULT:
            traffic_workload = args.config + "_packed"
    elif args.config == "c5":
        # tall and skinny: the GEMM streams P planes of A and B once (K x (M + N) bytes
        # each) and does little MFMA work per byte, so HBM bounds it
        gemm_bytes = P * K * (M + N) + P * M * N
        gbs = gemm_bytes / (stage[2] * 1e-3) / 1e9
        roofline = {"bound": "hbm", "kernel": kernel, "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(gbs / PEAK_HBM_GBS, 4), "per_launch_bytes": gemm_bytes}
        traffic_kernels, traffic_workload = ["plane_gemm_kernel", "residue_finalize_kernel"], "c5_packed"
    roofline["traffic"] = traffic_from_profiles(traffic_kernels, traffic_workload)
    if roofline["traffic"] is not None:
        roofline["traffic_source"] = ("profiles/traffic.json: rocprofv3 FETCH_SIZE and WRITE_SIZE per dispatch of "
                                      f"{' + '.join(traffic_kernels)} at this workload, copy-calibrated; not "
                                      "measured in this run")
    result = {
        "metric": metric,
        "value": round(value, 3),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int64 (int8 residue MFMA)",
        "data": (f"synthetic: SplitMix64 uniform [-2^{bits}, 2^{bits}) int64 operands, resident in HBM" if signed
                 else f"synthetic: SplitMix64 uniform [0, 2^{bits}) uint64 operands, resident in HBM"),
        "config": {
            "workload": workload,
            "m": M, "n": N, "k": K, "prefix": P, "bound": "per tile" if tiled else str(bound),
            "stage_ms": {"pack_a": round(stage[0], 4), "pack_b": round(stage[1], 4), "gemm": round(stage[2], 4),
                         "export": round(stage[3], 4)},
            "range_status": int(status[0]),
            "graph_replay": bool(graph),
            "settle_steps": args.settle_steps,
        },
        "roofline": roofline,
        "cpu_baseline": None,
    }
    if roofline["bound"] == "mfma":
        roofline["attainable"] = optional_probe(attainable_mfma, roofline["achieved"])
    if not fused:
        # the pack and export stages are memory-bound streams: report them
        # against a plain stream of the same reads and writes (those moving
        # at least 16 MB; smaller ones are launch-bound), each timed as the
        # probe is, over back-to-back launches after the stage pass (the
        # stage pass's events add a few us to every stage, a tenth of a pack)
        calls = {"pack_a": (8 * M * K, P * M * K, lambda: r.check(pack(ctx.ptr, Am.ptr, dA, K, 0, stream), "pack A")),
                 "pack_b": (8 * K * N, P * K * N, lambda: r.check(pack(ctx.ptr, Bm.ptr, dB, N, 0, stream), "pack B"))}
        if not tiled:
            calls["export"] = (P * M * N, 8 * M * N,
                               lambda: r.check(export(ctx.ptr, plan.ptr, Cm.ptr, dC, N, dS, stream), "export"))
        streams = {k: (rd, wr, back_to_back_ms(call, stream, args.steps)) for k, (rd, wr, call) in calls.items()
                   if rd + wr >= (16 << 20)}
        if streams:
            result["stage_streams"] = optional_probe(attainable_streams, streams)

    if tiled:
        # exact in int64 (|C| <= 2^62): sampled rows of every tile row against numpy
        rows = np.arange(0, M, TILED_EDGE // 2)
        want = A[rows].astype(np.int64) @ B.astype(np.int64)
        result["config"]["rows_bit_exact"] = bool(np.array_equal(Cout[rows], want))
        log(f"[bench] {len(rows)} sampled rows bit-exact: {result['config']['rows_bit_exact']}")
    elif not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args, A, B, Cout, P, bound, signed)

    print(json.dumps(result))
    if graph:
        hip.graph_destroy(*graph)
    for e in (start, stop):
        hip.event_destroy(e)
    hip.stream_destroy(stream)
    for p in (dA, dB, dC, dS):
        hip.free(p)
    if args.rns8_bench_json:
        write_v4_capture(args, ctx, A, B, signed, bound, budget, forced, tile_bounds if tiled else None)
    return 0


def write_v4_capture(args, ctx, A, B, signed, bound, budget, forced, tile_bounds) -> None:
    """The same GEMM through the public host-buffer ABI (pack from host arrays,
    rns8_gemm_rns, export to a host array; PCIe included), written as an
    rns8-bench schema-v4 record (rns8_amd/bench_v4.py)."""
    from rns8_amd import bench_v4

    bits = CONFIGS[args.config][4]
    dist = (f"splitmix64_{'signed' if signed else 'unsigned'}_uniform_2^{bits}"
            + ("_tile_rows_scaled" if tile_bounds is not None else ""))
    rec, _ = bench_v4.capture_bounded(
        ctx, A, B, signed=signed, bound=bound, budget=budget, forced=forced,
        tile_bounds_fn=(lambda: tile_bounds) if tile_bounds is not None else None, tile=TILED_EDGE,
        warmups=1, repeats=3, seed=args.seed, input_distribution=dist, command_line=" ".join(sys.argv))
    Path(args.rns8_bench_json).write_text(json.dumps(rec, indent=2) + "\n")
    log(f"[bench] schema-v4 capture: {args.rns8_bench_json} (host-API end to end "
        f"{rec['avg_end_to_end_us']:.0f} us, gemm {rec['avg_rns_gemm_us']:.0f} us)")


def cpu_baseline(args, A, B, Cout, P, bound, signed) -> dict:
    """The oracle's CPU_REFERENCE pipeline (pack A rows + pack all of B +
    per-plane int32 ring GEMM + Garner export; oracle/rns8_oracle.c) on rows
    [0, R) of the same GEMM, R sized so the timed run takes about
    --cpu-seconds. Two short calibration runs separate the fixed cost (packing
    B) from the per-row cost. The sampled rows are compared bit-exactly with
    the GPU result."""
    import oracle

    threads, share = cpu_share()
    oracle.set_threads(threads)
    run = oracle.gemm_i64 if signed else oracle.gemm_u64
    M, K = A.shape
    N = B.shape[1]

    def timed(rows):
        t0 = time.perf_counter()
        st, ref = run(A, B, P, bound, row0=0, rows=rows)
        return time.perf_counter() - t0, st, ref

    r1, r2 = 8, 40
    t1, _, _ = timed(r1)
    t2, _, _ = timed(r2)
    per_row = max((t2 - t1) / (r2 - r1), 1e-6)
    fixed = max(t1 - r1 * per_row, 0.0)
    rows = int((args.cpu_seconds - fixed) / per_row) if args.cpu_seconds > fixed else r2
    rows = max(r2, min(M, rows // 8 * 8))
    t_cpu, st, ref = timed(rows)
    match = bool(st == 0 and np.array_equal(ref, Cout[:rows]))
    reps = 1
    # the whole GEMM can take less than the target: repeat it and average
    while rows == M and reps * t_cpu < args.cpu_seconds and reps < 32:
        t_next, _, _ = timed(rows)
        t_cpu = (t_cpu * reps + t_next) / (reps + 1)
        reps += 1
    cpu_tops = 2.0 * rows * N * K / t_cpu / 1e12
    log(f"[bench] cpu baseline {cpu_tops:.5f} TOPS on {rows} rows in {t_cpu:.2f} s "
        f"(fixed {fixed:.2f} s, {1e3 * per_row:.1f} ms/row), match={match}")
    return {
        "value": round(cpu_tops, 6),
        "unit": "TOPS",
        "cores": threads,
        "cpu_share": share,
        "kind": "port",
        "sample": f"rows 0..{rows - 1} of C ({rows}x{N}x{K}, prefix {P}; pack of all of B included), "
                  f"{t_cpu:.2f} s per run, {reps} run(s), on {threads} threads of {_cpu_model()}",
        "rows_bit_exact_vs_gpu": match,
    }


def cpu_share() -> tuple[int, dict]:
    """Threads for the CPU baseline: the CPUs this process may run on
    (sched_getaffinity), capped by the cgroup CPU quota where one is set (a
    quota of Q CPUs gives at most Q threads' worth of time). Returns the
    thread count and what it was derived from."""
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    quota = None
    try:
        q, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            quota = int(q) / int(period)
    except (OSError, ValueError):
        pass
    threads = affinity if quota is None else max(1, min(affinity, int(quota)))
    return threads, {"nproc": os.cpu_count(), "affinity": affinity, "cgroup_quota_cpus": quota}


def grouped_bench(args) -> int:
    """GROUP_TASKS int64 GEMMs of one shape per step: pack every A_i and B_i,
    one rns8_mi355x_gemm_rns_grouped_async call, export every C_i, all on one
    stream. Also times the same GEMMs as GROUP_TASKS ungrouped calls."""
    import rns8_amd as r
    from rns8_amd import hip, inputs

    _, M, N, K, bits, bound, budget, forced = GROUPED
    T = GROUP_TASKS
    log(f"[bench] grouped: {T} x int64 {M}x{N}x{K} bits={bits}")
    ctx = r.Context()
    bk = r.BOUND_GLOBAL_MAX_ABS
    desc = r.gemm_desc(r.BOUNDED_I64, bk, M, N, K, bound=bound, max_prefix=budget,
                       flags=r.PLAN_FORCE_FIXED_PREFIX if forced else 0)
    plan = r.Plan(ctx, desc)
    P = plan.prefix
    mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, r.BOUNDED_I64, bk, P))
    quads = [(mk(M, K), mk(K, N), mk(M, N), r.Workspace(ctx, plan)) for _ in range(T)]
    tasks = r.grouped_tasks(quads)
    host = [(inputs.int_range(inputs.operand_seed(args.seed + i, "A"), (M, K), bits),
             inputs.int_range(inputs.operand_seed(args.seed + i, "B"), (K, N), bits)) for i in range(T)]
    dev = []
    for A, B in host:
        dA, dB, dC = hip.malloc(A.nbytes), hip.malloc(B.nbytes), hip.malloc(M * N * 8)
        hip.to_device(dA, A)
        hip.to_device(dB, B)
        dev.append((dA, dB, dC))
    dS = hip.malloc(64)
    hip.memset(dS, 0, 64)
    stream = hip.stream_create()
    L = r.lib()
    def step(mark=_no_mark, grouped: bool = True):
        mark(0)
        for (Am, Bm, _, _), (dA, dB, _) in zip(quads, dev):
            r.check(L.rns8_mi355x_pack_i64_device(ctx.ptr, Am.ptr, dA, K, 0, stream), "pack A")
            r.check(L.rns8_mi355x_pack_i64_device(ctx.ptr, Bm.ptr, dB, N, 0, stream), "pack B")
        mark(1)
        if grouped:
            r.check(L.rns8_mi355x_gemm_rns_grouped_async(ctx.ptr, plan.ptr, tasks, T, stream), "grouped gemm")
        else:
            for Am, Bm, Cm, ws in quads:
                r.check(L.rns8_mi355x_gemm_rns_async(ctx.ptr, plan.ptr, Am.ptr, Bm.ptr, Cm.ptr, ws.ptr, stream),
                        "gemm")
        mark(2)
        for (_, _, Cm, _), (_, _, dC) in zip(quads, dev):
            r.check(L.rns8_mi355x_export_i64_device(ctx.ptr, plan.ptr, Cm.ptr, dC, N, dS, stream), "export")
        mark(3)

    settle(step, args.settle_steps, hip.synchronize)
    for _ in range(args.warmup):
        step()
    hip.synchronize()
    start, stop = hip.event_create(), hip.event_create()
    hip.event_record(start, stream)
    for _ in range(args.steps):
        step()
    hip.event_record(stop, stream)
    hip.stream_synchronize(stream)
    ms_per_step = hip.event_elapsed_ms(start, stop) / args.steps
    # stage timing, after the timed pass: grouped and ungrouped steps back to
    # back, alternating
    timer, timer_ungrouped = StageTimer(args.steps, 4, stream), StageTimer(args.steps, 4, stream)
    for s in range(args.steps):
        step(timer.marker(s))
        step(timer_ungrouped.marker(s), grouped=False)
    stage = timer.stage_ms()
    ungrouped = timer_ungrouped.stage_ms()[1]
    timer.destroy()
    timer_ungrouped.destroy()
    log(f"[bench] stage ms: pack {stage[0]:.4f} grouped gemm {stage[1]:.4f} export {stage[2]:.4f}; "
        f"{T} ungrouped gemms {ungrouped:.4f}")
    status = np.zeros(16, dtype=np.uint32)
    hip.from_device(status, dS)
    out = np.empty((M, N), dtype=np.int64)
    hip.from_device(out, dev[-1][2])
    rows = np.arange(0, M, 64)
    exact = bool(np.array_equal(out[rows], host[-1][0][rows] @ host[-1][1]))
    log(f"[bench] {ms_per_step:.4f} ms per step; last task's sampled rows exact: {exact}")
    ops = 2.0 * M * N * K * T
    gemm_ops = ops * P
    achieved = gemm_ops / (stage[1] * 1e-3) / 1e12
    result = {
        "metric": "exact int64 grouped GEMM effective TOPS (2MNK*tasks/s)",
        "value": round(ops / (ms_per_step * 1e-3) / 1e12, 3), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int64 (int8 residue MFMA)",
        "data": f"synthetic: SplitMix64 uniform [-2^{bits}, 2^{bits}) int64 operands, resident in HBM",
        "config": {"workload": f"{T} x RNS8_BOUNDED_I64 {M}x{N}x{K} prefix {P} (FORCE_FIXED_PREFIX), pack + "
                               "rns8_gemm_rns_grouped + export device-resident",
                   "tasks": T, "m": M, "n": N, "k": K, "prefix": P,
                   "stage_ms": {"pack": round(stage[0], 4), "grouped_gemm": round(stage[1], 4),
                                "export": round(stage[2], 4), "ungrouped_gemms": round(ungrouped, 4)},
                   "range_status": int(status[0]), "rows_bit_exact": exact, "settle_steps": args.settle_steps},
        "roofline": {"bound": "mfma", "kernel": "plane_gemm_kernel<Cfg<4,4>,1,true,false,true> (grouped, persistent)",
                     "achieved": round(achieved, 2), "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                     "frac": round(achieved / PEAK_INT8_TOPS, 4), "traffic": None, "per_launch_ops": gemm_ops},
        "cpu_baseline": None,
    }
    result["roofline"]["attainable"] = optional_probe(attainable_mfma, achieved)
    print(json.dumps(result))
    for e in (start, stop):
        hip.event_destroy(e)
    hip.stream_destroy(stream)
    for d in dev:
        for p in d:
            hip.free(p)
    hip.free(dS)
    return 0


def finite_or_wide_bench(args) -> int:
    """C2 (finite field 251, 4096^3 uint8, one plane) or C4 (exact-wide signed,
    2048^3 full-range int64, prefix 20 forced, 3-limb export): pack A, pack B,
    GEMM, export per step through the device entry points on one stream."""
    import rns8_amd as r
    from rns8_amd import hip, inputs

    finite = args.config == "c2"
    if finite:
        M = N = K = 4096
        P, modulus = 1, 251
        sem, bk = r.FINITE_FIELD_U8, r.BOUND_NONE
        desc = r.gemm_desc(sem, bk, M, N, K, finite_modulus=modulus)
        A = inputs.bytes_below(inputs.operand_seed(args.seed, "A"), (M, K), modulus)
        B = inputs.bytes_below(inputs.operand_seed(args.seed, "B"), (K, N), modulus)
        elem = 1
    else:
        M = N = K = 2048
        modulus, limbs = 0, 3
        sem, bk = r.EXACT_WIDE_SIGNED, r.BOUND_NONE
        desc = r.gemm_desc(sem, bk, M, N, K, max_prefix=20, flags=r.PLAN_FORCE_FIXED_PREFIX)
        A = inputs.full_int64(inputs.operand_seed(args.seed, "A"), (M, K))
        B = inputs.full_int64(inputs.operand_seed(args.seed, "B"), (K, N))
        elem = 8 * limbs
    log(f"[bench] config {args.config}: {M}x{N}x{K}")
    ctx = r.Context()
    plan = r.Plan(ctx, desc)
    if not finite:
        P = plan.prefix
    mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, bk, 0 if finite else P))
    Am, Bm, Cm = mk(M, K), mk(K, N), mk(M, N)
    ws = r.Workspace(ctx, plan)
    dA, dB, dC, dS = hip.malloc(A.nbytes), hip.malloc(B.nbytes), hip.malloc(M * N * elem), hip.malloc(64)
    hip.to_device(dA, A)
    hip.to_device(dB, B)
    hip.memset(dS, 0, 64)
    stream = hip.stream_create()
    L = r.lib()
    def step(mark=_no_mark):
        mark(0)
        if finite:
            r.check(L.rns8_mi355x_pack_finite_u8_device(ctx.ptr, Am.ptr, modulus, dA, K, 0, stream), "pack A")
        else:
            r.check(L.rns8_mi355x_pack_i64_device(ctx.ptr, Am.ptr, dA, K, 0, stream), "pack A")
        mark(1)
        if finite:
            r.check(L.rns8_mi355x_pack_finite_u8_device(ctx.ptr, Bm.ptr, modulus, dB, N, 0, stream), "pack B")
        else:
            r.check(L.rns8_mi355x_pack_i64_device(ctx.ptr, Bm.ptr, dB, N, 0, stream), "pack B")
        mark(2)
        if finite:
            r.check(L.rns8_mi355x_gemm_finite_u8_async(ctx.ptr, plan.ptr, modulus, Am.ptr, Bm.ptr, Cm.ptr, ws.ptr,
                                                        stream), "gemm")
        else:
            r.check(L.rns8_mi355x_gemm_rns_async(ctx.ptr, plan.ptr, Am.ptr, Bm.ptr, Cm.ptr, ws.ptr, stream), "gemm")
        mark(3)
        if finite:
            r.check(L.rns8_mi355x_export_finite_u8_device(ctx.ptr, plan.ptr, modulus, Cm.ptr, dC, N, stream), "export")
        else:
            r.check(L.rns8_mi355x_export_exact_wide_signed_limbs_device(ctx.ptr, plan.ptr, Cm.ptr, dC, N, limbs, dS,
                                                                        stream), "export")
        mark(4)

    settle(step, args.settle_steps, hip.synchronize)
    for _ in range(args.warmup):
        step()
    hip.synchronize()
    start, stop = hip.event_create(), hip.event_create()
    hip.event_record(start, stream)
    for _ in range(args.steps):
        step()
    hip.event_record(stop, stream)
    hip.stream_synchronize(stream)
    ms_per_step = hip.event_elapsed_ms(start, stop) / args.steps
    # stage timing, after the timed pass
    timer = StageTimer(args.steps, 5, stream)
    for s in range(args.steps):
        step(timer.marker(s))
    stage = timer.stage_ms()
    timer.destroy()
    log(f"[bench] stage ms: packA {stage[0]:.4f} packB {stage[1]:.4f} gemm {stage[2]:.4f} export {stage[3]:.4f}")
    rows = np.arange(0, M, M // 16)
    if finite:
        out = np.empty((M, N), dtype=np.uint8)
        hip.from_device(out, dC)
        want = (A[rows].astype(np.int64) @ B.astype(np.int64)) % modulus
        exact = bool(np.array_equal(out[rows], want))
    else:
        out = np.empty((M, N * limbs), dtype=np.uint64)
        hip.from_device(out, dC)
        rows = rows[:4]
        Ao, Bo = A[rows].astype(object), B.astype(object)

        def value(i, j):  # little-endian two's-complement limbs -> Python int
            v = sum(int(w) << (64 * l) for l, w in enumerate(out[i, limbs * j:limbs * j + limbs]))
            return v - (1 << (64 * limbs)) if v >> (64 * limbs - 1) else v

        exact = all(value(i, j) == int((Ao[t] * Bo[:, j]).sum()) for t, i in enumerate(rows)
                    for j in (0, 1, N // 2, N - 1))
    status = np.zeros(16, dtype=np.uint32)
    hip.from_device(status, dS)
    log(f"[bench] {ms_per_step:.4f} ms per step; sampled outputs exact: {exact}")
    ops = 2.0 * M * N * K
    achieved = ops * P / (stage[2] * 1e-3) / 1e12
    result = {
        "metric": (f"exact finite-field u8 GEMM mod {modulus} effective TOPS at 4096\u00b3" if finite else
                   f"exact-wide signed GEMM effective TOPS (2MNK/s) at 2048\u00b3 prefix {P}, 3-limb export"),
        "value": round(ops / (ms_per_step * 1e-3) / 1e12, 3), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u8" if finite else "int64 (int8 residue MFMA)",
        "data": ("synthetic: SplitMix64 uniform [0, 251) uint8 operands" if finite else
                 "synthetic: SplitMix64 full-range int64 operands") + ", resident in HBM",
        "config": {"workload": f"{args.config} {M}x{N}x{K} prefix {P}, pack+GEMM+export device-resident",
                   "m": M, "n": N, "k": K, "prefix": P,
                   "stage_ms": {"pack_a": round(stage[0], 4), "pack_b": round(stage[1], 4),
                                "gemm": round(stage[2], 4), "export": round(stage[3], 4)},
                   "range_status": int(status[0]), "sampled_outputs_exact": exact,
                   "settle_steps": args.settle_steps},
        "roofline": {"bound": "mfma", "kernel": "plane_gemm_kernel<Cfg<4,4>,1,true,false,false> (256x256 tiles, persistent)",
                     "achieved": round(achieved, 2), "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                     "frac": round(achieved / PEAK_INT8_TOPS, 4), "traffic": None, "per_launch_ops": ops * P},
        "cpu_baseline": None,
    }
    result["roofline"]["attainable"] = optional_probe(attainable_mfma, achieved)
    print(json.dumps(result))
    for e in (start, stop):
        hip.event_destroy(e)
    hip.stream_destroy(stream)
    for p_ in (dA, dB, dC, dS):
        hip.free(p_)
    return 0


def tiled_operands(A, bits, N, K):
    """A with its 128-row blocks scaled to |a| <= 2^TILED_ROW_BITS[i % 7]
    (arithmetic shift of the 2^bits operand), and the per-tile bounds
    K * 2^row_bits * 2^bits (|b| <= 2^bits), row-major over 128 x 128 tiles."""
    A = A.copy()
    tiles_m, tiles_n = -(-A.shape[0] // TILED_EDGE), -(-N // TILED_EDGE)
    bounds = []
    for t in range(tiles_m):
        row_bits = TILED_ROW_BITS[t % len(TILED_ROW_BITS)]
        A[t * TILED_EDGE:(t + 1) * TILED_EDGE] >>= bits - row_bits
        bounds += [K << (row_bits + bits)] * tiles_n
    return A, bounds


def traffic_from_profiles(kernels, workload: str):
    """HBM bytes per launch of the timed kernel (or the sum over the kernels
    of one timed stage) from the committed rocprofv3 counter summary
    (profiles/traffic.json: FETCH_SIZE and WRITE_SIZE per dispatch, scaled by
    a device-copy calibration of known size), or None."""
    path = ROOT / "profiles" / "traffic.json"
    if isinstance(kernels, str):
        kernels = [kernels]
    try:
        data = json.loads(path.read_text())
        return sum(int(data["kernels"][workload][k]["hbm_bytes_per_launch"]) for k in kernels)
    except (OSError, KeyError, ValueError):
        return None


def copy_calibration(nbytes: int, reps: int) -> int:
    """Plain device-to-device copy kernel of known size (for scaling the
    FETCH_SIZE / WRITE_SIZE counters); prints bytes and time per copy."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / reps
    print(json.dumps({"copy_bytes": nbytes, "reps": reps, "ms_per_copy": round(dt * 1e3, 4),
                      "GBps_read_plus_write": round(2 * nbytes / dt / 1e9, 1)}))
    return 0


def oneshot_rate(args) -> int:
    """rns8_gemm_i64_oneshot / rns8_gemm_u64_oneshot on host arrays: H2D of A
    and B, pack, GEMM, export and D2H of C per call (the reference's oneshot
    contract, api_oneshot.cpp:510-586). Prints one JSON line; this rate is
    reported beside the HBM-resident figure, never as `value`."""
    import rns8_amd as r
    from rns8_amd import inputs

    sem, M, N, K, bits, bound, budget, forced = CONFIGS[args.config]
    signed = sem == "i64"
    gen = inputs.int_range if signed else inputs.uint_range
    A = gen(inputs.operand_seed(args.seed, "A"), (M, K), bits)
    B = gen(inputs.operand_seed(args.seed, "B"), (K, N), bits)
    desc = r.gemm_desc(r.BOUNDED_I64 if signed else r.BOUNDED_U64,
                       r.BOUND_GLOBAL_MAX_ABS if signed else r.BOUND_GLOBAL_MAX_UNSIGNED, M, N, K, bound=bound,
                       max_prefix=budget, flags=r.PLAN_FORCE_FIXED_PREFIX if forced else 0)
    fn = r.gemm_i64_oneshot if signed else r.gemm_u64_oneshot
    C = np.zeros((M, N), dtype=np.int64 if signed else np.uint64)
    with r.Context() as ctx:
        for _ in range(max(args.warmup, 1)):
            st, _ = fn(ctx, desc, A, B, C)
            r.check(st, "oneshot")
        t0 = time.perf_counter()
        for _ in range(args.steps):
            st, _ = fn(ctx, desc, A, B, C)
        dt = (time.perf_counter() - t0) / args.steps
        r.check(st, "oneshot")
    print(json.dumps({"mode": "oneshot (host buffers, PCIe included)", "config": args.config, "m": M, "n": N,
                      "k": K, "ms_per_call": round(dt * 1e3, 3),
                      "effective_TOPS": round(2.0 * M * N * K / dt / 1e12, 3),
                      "host_bytes_moved": int(A.nbytes + B.nbytes + C.nbytes)}))
    return 0


def host_pack_rate(args) -> int:
    """The public host-array entries on C4's exact-wide operands (2048 x 2048
    full-range int64, prefix 20): rns8_pack_i64 uploads the array, proves its
    range on the device (per-row and per-column summaries, exact_axes.hip)
    and packs it; rns8_gemm_rns admits the product (on k maxA maxB, which
    fits at prefix 20). Times both against a bare upload of the same bytes,
    and the admission that needs the refined bound: D = C x B with C the
    result above, whose worst case does not fit, so the call computes C's
    summaries and D's cell bounds on the device (2 x 2048^2 cells) and reads
    the bound back (the product is then refused, as the reference refuses
    it). Prints one JSON line; not a `value`."""
    import rns8_amd as r
    from rns8_amd import hip, inputs

    n = 2048
    A = inputs.full_int64(inputs.operand_seed(args.seed, "A"), (n, n))
    B = inputs.full_int64(inputs.operand_seed(args.seed, "B"), (n, n))
    with r.Context() as ctx:
        desc = r.gemm_desc(r.EXACT_WIDE_SIGNED, r.BOUND_NONE, n, n, n, max_prefix=20, flags=r.PLAN_FORCE_FIXED_PREFIX)
        plan = r.Plan(ctx, desc)
        mk = lambda: r.Matrix(ctx, r.matrix_desc(n, n, r.EXACT_WIDE_SIGNED, r.BOUND_NONE, plan.prefix))
        Am, Bm, Cm = mk(), mk(), mk()
        ws = r.Workspace(ctx, plan)
        d = hip.malloc(A.nbytes)
        reps = max(args.steps, 1)

        def timed(fn):
            for _ in range(2):
                fn()
            hip.synchronize()
            t0 = time.perf_counter()
            for _ in range(reps):
                fn()
            hip.synchronize()
            return (time.perf_counter() - t0) / reps * 1e3

        upload = timed(lambda: hip.to_device(d, A))
        # source version 0: every call packs (a matrix given the source
        # version it already holds skips the pack)
        flip = [0]

        def packs():
            x, y = (A, B) if flip[0] == 0 else (B, A)
            flip[0] ^= 1
            r.check(r.pack_i64(ctx, Am, x, 0), "pack A")
            r.check(r.pack_i64(ctx, Bm, y, 0), "pack B")

        pack = timed(packs)
        gemm = timed(lambda: r.check(r.gemm_rns(ctx, plan, Am, Bm, Cm, ws), "gemm"))
        Dm = mk()

        def refused_chain():
            # C is a fresh lazy result each time, so each call computes C's summaries too
            r.check(r.lib().rns8_mi355x_gemm_rns_async(ctx.ptr, plan.ptr, Am.ptr, Bm.ptr, Cm.ptr, ws.ptr, None), "C")
            st = r.gemm_rns(ctx, plan, Cm, Bm, Dm, ws)
            if st != r.RANGE_ERROR:
                raise RuntimeError(f"chain status {st}, expected RNS8_RANGE_ERROR")

        chain = timed(refused_chain)
        hip.free(d)
    print(json.dumps({"mode": "exact-wide host-array packs and GEMM (C4 operands, public ABI)", "n": n,
                      "prefix": plan.prefix, "ms_upload_one_operand": round(upload, 3),
                      "ms_pack_two_operands": round(pack, 3), "ms_gemm_rns_with_admission": round(gemm, 3),
                      "ms_gemm_plus_refined_admission": round(chain, 3)}))
    return 0


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    sys.exit(main())
