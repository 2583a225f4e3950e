"""rns8-bench schema-v4 capture records for the bounded persistent-RNS lane.

The reference's benchmark driver (benchmarks/rns8_bench.cpp and its
rns8_bench_print_json*.inc sections) writes one JSON object per run; its
schema package (tools/benchmark_schema/core_shared.py:39-55) fixes the version
(4), the timing phases and their repeat rules. This module produces the same
record for the bounded int64 / uint64 lane ("rns8_bounded_gemm_persistent_rns":
plan, schedule query, matrix allocation once; then per repeat pack A and B
from host arrays, rns8_gemm_rns, export to a host array), timed with the host
clock around the public C ABI calls, as the reference's lane is
(rns8_bench_bounded_i64_lane.inc). Captures from this library can therefore
sit beside the reference's gfx1100 records.

Differences kept visible in the record: the input generator is SplitMix64
(`input_distribution` says so), so checksums match only captures made from
the same inputs; HIP event timing is not collected in this lane
(`gpu_event_timing` false, its fields null, as the schema requires).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import time

import numpy as np

from . import abi

SCHEMA_VERSION = 4
TIMING_PHASES = ["planning", "scheduling", "matrix_alloc", "pack", "rns_gemm", "crt_export", "end_to_end"]
PER_TILE_PHASE = "tile_bound_scan"
REPEATED_PHASES = {"pack", "rns_gemm", "crt_export", "end_to_end"}
FNV_OFFSET = 1469598103934665603
FNV_PRIME = 1099511628211


def percentile(values, p: float) -> float:
    """The schema's percentile: the element at ceil-ish index p * (n - 1) of the
    sorted values (tools/benchmark_schema/core_shared.py:319-324)."""
    if not values:
        return 0.0
    ordered = sorted(values)
    return float(ordered[int(p * float(len(ordered) - 1) + 0.999999)])


def summary(values) -> dict:
    return {"avg": sum(values) / len(values) if values else 0.0, "median": percentile(values, 0.50),
            "p95": percentile(values, 0.95)}


def checksum_u64(values: np.ndarray) -> int:
    """FNV-1a over the 64-bit words of a row-major matrix, one word per step
    (the reference's checksum_matrix, rns8_bench_event_phase_helpers.inc:544-552,
    mix_checksum rns8_bench_support.cpp:96-99). A sequential fold: about 8 s
    for 4096 x 4096 words."""
    words = np.ascontiguousarray(values).view(np.uint64).reshape(-1)
    h = FNV_OFFSET
    prime = FNV_PRIME
    mask = (1 << 64) - 1
    for w in words.tolist():
        h = ((h ^ w) * prime) & mask
    return h


def _us(t0: int, t1: int) -> int:
    return max(0, (t1 - t0) // 1000)


def _text(b: bytes) -> str:
    return b.decode("ascii", "replace")


def _hipcc_version() -> str:
    try:
        out = subprocess.run(["/opt/rocm/bin/hipcc", "--version"], capture_output=True, text=True, timeout=30)
        return " | ".join(line.strip() for line in out.stdout.splitlines()[:3] if line.strip())
    except (OSError, subprocess.SubprocessError):
        return "unknown"


def build_record(*, semantics: str, bound_kind: str, bound_mode: str, bound: int, m: int, n: int, k: int,
                 prefix: int, tile_m: int, tile_n: int, k_block_size: int, tile_bounds: list | None,
                 schedule: dict, backend: dict, seed: int, warmups: int, repeats: int, input_distribution: str,
                 command_line: str, device: dict, raw: dict, checksum: int, git_commit: str = "unknown") -> dict:
    """Assembles a capture from measured timings (microseconds, integers) and
    metadata; pure, so the record layout is testable without a device."""
    phases = list(TIMING_PHASES)
    if bound_mode == "per_tile":
        phases.insert(phases.index("matrix_alloc"), PER_TILE_PHASE)
    for p in phases:
        want = repeats if p in REPEATED_PHASES else 1
        if len(raw.get(p, [])) != want:
            raise ValueError(f"phase {p}: {len(raw.get(p, []))} values, expected {want}")
    avg = {p: sum(raw[p]) / len(raw[p]) for p in phases}
    per_modulus = prefix > 0
    notes = {
        "planning": "one-time rns8_create_plan plus rns8_create_workspace host timing",
        "scheduling": "one-time rns8_get_plan_schedule_info host timing",
        "matrix_alloc": "one-time persistent matrix allocation host timing",
        "pack": "per-repeat host timing for packing A and B from host arrays into persistent RNS matrices",
        "rns_gemm": "per-repeat host timing for rns8_gemm_rns",
        "crt_export": "per-repeat host timing for export/reconstruction into a host array",
        "end_to_end": "per-repeat pack plus rns_gemm plus crt_export host timing",
    }
    availability = {
        "scheduling": {"timed": True, "timing_key": "scheduling", "scope": "one_time_schedule_info_query",
                       "reason": "measured with the host clock around rns8_get_plan_schedule_info"},
        "reduction": {"timed": False, "timing_key": None, "scope": "fused_into_rns_gemm",
                      "reason": "the plane GEMM reduces to centered residues in its epilogue, so no separate "
                                "reduction kernel exists"},
    }
    if bound_mode == "per_tile":
        notes[PER_TILE_PHASE] = "one-time per-output-tile bound computation before plan creation"
        availability[PER_TILE_PHASE] = {"timed": True, "timing_key": PER_TILE_PHASE,
                                        "scope": "exact_seeded_input_prepass",
                                        "reason": "measured with the host clock around the per-tile bound "
                                                  "computation"}
    rec = {
        "schema_version": SCHEMA_VERSION,
        "benchmark": "rns8_bounded_gemm_persistent_rns",
        "backend_requested": "hip-direct",
        "backend_selected": "hip-direct",
        "selected_kernel": backend["selected_kernel"],
        "backend_metadata": backend,
        "semantics": semantics,
        "bound_kind": bound_kind,
        "bound_mode": bound_mode,
        "bound": int(bound),
        "m": m, "n": n, "k": k, "prefix": prefix, "tile_m": tile_m, "tile_n": tile_n,
        "layout": "row_major",
        "k_block_size": k_block_size,
        "adaptive_tile_size": None,
        "tile_bounds_u64": None if tile_bounds is None else {
            "source": "seeded_input_magnitude_bound", "pattern": "row_block_magnitude_times_k",
            "order": "row_major_output_tiles", "count": len(tile_bounds), "min": int(min(tile_bounds)),
            "max": int(max(tile_bounds)), "hash_u64": checksum_u64(np.array(tile_bounds, dtype=np.uint64))},
        "schedule_metadata": schedule,
        "epilogue_type": "crt_export",
        "packed_layout_version": None,
        "seed": seed, "warmups": warmups, "repeats": repeats,
        "input_distribution": input_distribution,
        "command_line": command_line,
        "git_commit": git_commit,
        "compiler": {"id": "hipcc", "version": _hipcc_version()},
        "configured_amdgpu_targets": "gfx950",
        "hip_toolchain": {"enabled": True, "hip_root": "/opt/rocm", "hipcc_path": "/opt/rocm/bin/hipcc",
                          "hipcc_version": _hipcc_version(), "hip_sdk_or_rocm_version": _rocm_version(),
                          "version_source": "hipcc --version"},
        "device": device,
        "clock_power_settings": None,
        "comparison_baseline": {
            "status": "required_not_recorded", "speedup_claimed": False, "selected_reference": None,
            "required_before_speedup_claim": ["same_contract_cpu_reference", "same_contract_direct_hip_correctness"],
            "reason": "raw capture; no same-contract baseline capture is attached"},
        "derived_tops_equivalent": None,
        "timing_source": "time.perf_counter_ns",
        "timing_note": "host wall-clock timings around the public C ABI calls of the gfx950 direct-HIP path",
        "timing_metadata": {
            "unit": "microseconds", "source": "time.perf_counter_ns", "source_scope": "host_wall_clock",
            "gpu_event_timing": False, "gpu_event_timing_reason": "not_collected_in_host_api_lane",
            "gpu_event_timing_status": "unavailable", "gpu_event_timing_source": None,
            "gpu_event_timing_source_scope": None, "gpu_event_timing_caveat": None,
            "phase_order": phases, "gpu_event_phase_order": None, "phase_notes": notes,
            "phase_availability": availability},
        "gpu_event_timings_us": None,
        "gpu_event_timing_summary_us": None,
        "plan_us": raw["planning"][0], "avg_planning_us": avg["planning"],
        "schedule_query_us": raw["scheduling"][0], "avg_scheduling_us": avg["scheduling"],
    }
    if bound_mode == "per_tile":
        rec["tile_bound_scan_us"] = raw[PER_TILE_PHASE][0]
        rec["avg_tile_bound_scan_us"] = avg[PER_TILE_PHASE]
    rec.update({
        "matrix_alloc_us": raw["matrix_alloc"][0], "avg_matrix_alloc_us": avg["matrix_alloc"],
        "avg_pack_us": avg["pack"], "avg_rns_gemm_us": avg["rns_gemm"],
        "per_modulus_gemm_estimate_applicable": per_modulus,
        "avg_per_modulus_gemm_estimate_us": round(avg["rns_gemm"] / prefix, 4) if per_modulus else None,
        "avg_crt_export_us": avg["crt_export"], "avg_end_to_end_us": avg["end_to_end"],
        "raw_timings_us": {p: [int(v) for v in raw[p]] for p in phases},
        "timing_summary_us": {p: summary(raw[p]) for p in phases},
        "checksum_u64": int(checksum),
    })
    return rec


def _rocm_version() -> str:
    try:
        with open("/opt/rocm/.info/version") as f:
            return f.read().strip()
    except OSError:
        return "unknown"


def backend_metadata(plan, semantics: str, m: int, n: int, k: int, prefix: int, tile_m: int, tile_n: int) -> dict:
    """rns8_get_plan_backend_info of the plan, in the capture's layout."""
    from . import lib

    info = abi.new_struct(abi.PlanBackendInfo)
    st = lib().rns8_get_plan_backend_info(plan.ptr, C.byref(info))
    if st != abi.SUCCESS:
        raise RuntimeError(f"rns8_get_plan_backend_info: status {st}")
    kernel = _text(info.selected_kernel)
    return {
        "source": "rns8_get_plan_backend_info",
        "selected_kernel": kernel,
        "accelerator_backend": bool(info.is_accelerator),
        "correctness_backend": bool(info.is_correctness_backend),
        "matrix_engine_backend": bool(info.is_matrix_engine_backend),
        "compiled_kernel_available": bool(info.compiled_kernel_available),
        "exact_differential_validated": bool(info.exact_differential_validated),
        "performance_validated": bool(info.performance_validated),
        "accelerator_library": _text(info.accelerator_library),
        "accelerator_version": None,
        "capability_status": _text(info.capability_status),
        "epilogue_mode": _text(info.epilogue_mode),
        "workspace_mode": _text(info.workspace_mode),
        "workspace_required_bytes": int(info.workspace_required_bytes),
        "isa_evidence": _text(info.isa_evidence),
        "autotune_key": (f"backend=hip-direct;target_id=gfx950;semantics={semantics};m={m};n={n};k={k};"
                         f"prefix={prefix};tile_m={tile_m};tile_n={tile_n};kernel={kernel}"),
        "accumulator_safety": {
            "input_domain": _text(info.accumulator_input_domain),
            "signedness": _text(info.accumulator_signedness),
            "accumulator_type": _text(info.accumulator_type),
            "modulus_policy": _text(info.accumulator_modulus_policy),
            "modulus": int(info.accumulator_modulus),
            "uses_int32_inner_product": bool(info.accumulator_uses_int32_inner_product),
            "k_block_size": int(info.accumulator_k_block_size),
            "k_block_cap": int(info.accumulator_k_block_cap),
            "max_lhs_abs": int(info.accumulator_max_lhs_abs),
            "max_rhs_abs": int(info.accumulator_max_rhs_abs),
            "max_product": int(info.accumulator_max_product),
            "safe_for_k_block": bool(info.accumulator_safe_for_k_block),
            "status": _text(info.accumulator_safety_status),
        },
    }


def schedule_metadata(plan) -> dict:
    s = plan.schedule_info()
    return {
        "source": "rns8_get_plan_schedule_info", "tile_m": s.tile_m, "tile_n": s.tile_n,
        "tile_rows": s.tile_rows, "tile_cols": s.tile_cols, "tile_count": s.tile_count,
        "min_required_prefix": s.min_required_prefix, "max_required_prefix": s.max_required_prefix,
        "min_selected_prefix": s.min_selected_prefix, "max_selected_prefix": s.max_selected_prefix,
        "prefix_group_count": s.prefix_group_count, "adaptive_prefix_active": bool(s.adaptive_prefix_active),
        "adaptive_skip_active": bool(s.adaptive_skip_active),
        "adaptive_execution_applied": bool(s.adaptive_prefix_active or s.adaptive_skip_active),
        "range_bit_length": s.range_bit_length,
        "zero_a_row_proof_count": s.zero_a_row_count, "zero_b_col_proof_count": s.zero_b_col_count,
        "zero_row_col_product_count": s.zero_row_col_product_count,
        "planner_zero_a_row_count": s.zero_a_row_count, "planner_zero_b_col_count": s.zero_b_col_count,
        "planner_zero_row_col_product_count": s.zero_row_col_product_count,
    }


def capture_bounded(ctx, A: np.ndarray, B: np.ndarray, *, signed: bool, bound: int = 0, budget: int = 0,
                    forced: bool = False, tile_bounds_fn=None, tile: int = 128, warmups: int = 1, repeats: int = 3,
                    seed: int = 0, input_distribution: str = "", command_line: str = "") -> tuple[dict, np.ndarray]:
    """Runs the lane on host operands A (m x k) and B (k x n) and returns
    (record, C). `tile_bounds_fn()` (per-tile mode) returns the row-major tile
    bounds and is timed as the tile-bound scan."""
    from . import (BOUND_GLOBAL_MAX_ABS, BOUND_GLOBAL_MAX_UNSIGNED, BOUND_PER_TILE_MAX_ABS,
                   BOUND_PER_TILE_MAX_UNSIGNED, BOUNDED_I64, BOUNDED_U64, PLAN_FORCE_FIXED_PREFIX, Matrix, Plan,
                   Workspace, check, export_i64, export_u64, gemm_desc, gemm_rns, matrix_desc, pack_i64, pack_u64)

    m, k = A.shape
    n = B.shape[1]
    sem = BOUNDED_I64 if signed else BOUNDED_U64
    per_tile = tile_bounds_fn is not None
    raw: dict[str, list[int]] = {}
    tile_bounds = None
    if per_tile:
        t0 = time.perf_counter_ns()
        tile_bounds = tile_bounds_fn()
        raw[PER_TILE_PHASE] = [_us(t0, time.perf_counter_ns())]
        bk = BOUND_PER_TILE_MAX_ABS if signed else BOUND_PER_TILE_MAX_UNSIGNED
        desc = gemm_desc(sem, bk, m, n, k, max_prefix=budget, flags=PLAN_FORCE_FIXED_PREFIX if forced else 0,
                         tile_m=tile, tile_n=tile, tile_bounds=tile_bounds)
    else:
        bk = BOUND_GLOBAL_MAX_ABS if signed else BOUND_GLOBAL_MAX_UNSIGNED
        desc = gemm_desc(sem, bk, m, n, k, bound=bound, max_prefix=budget,
                         flags=PLAN_FORCE_FIXED_PREFIX if forced else 0)
    t0 = time.perf_counter_ns()
    plan = Plan(ctx, desc)
    ws = Workspace(ctx, plan)
    raw["planning"] = [_us(t0, time.perf_counter_ns())]
    t0 = time.perf_counter_ns()
    schedule = schedule_metadata(plan)
    raw["scheduling"] = [_us(t0, time.perf_counter_ns())]
    prefix = schedule["max_selected_prefix"]
    tm, tn = (tile, tile) if per_tile else (schedule["tile_m"], schedule["tile_n"])
    t0 = time.perf_counter_ns()
    mk = lambda rows, cols: Matrix(ctx, matrix_desc(rows, cols, sem, bk, prefix, tile_m=tm if per_tile else 0,
                                                    tile_n=tn if per_tile else 0))
    Am, Bm, Cm = mk(m, k), mk(k, n), mk(m, n)
    raw["matrix_alloc"] = [_us(t0, time.perf_counter_ns())]
    pack = pack_i64 if signed else pack_u64
    export = export_i64 if signed else export_u64
    out = np.zeros((m, n), dtype=np.int64 if signed else np.uint64)
    for p in REPEATED_PHASES:
        raw[p] = []
    for rep in range(warmups + repeats):
        t0 = time.perf_counter_ns()
        # a new source version per repeat, so the pack is never elided
        check(pack(ctx, Am, A, 2 * rep + 1), "pack A")
        check(pack(ctx, Bm, B, 2 * rep + 2), "pack B")
        t1 = time.perf_counter_ns()
        check(gemm_rns(ctx, plan, Am, Bm, Cm, ws), "rns8_gemm_rns")
        t2 = time.perf_counter_ns()
        check(export(ctx, plan, Cm, out), "export")
        t3 = time.perf_counter_ns()
        if rep >= warmups:
            raw["pack"].append(_us(t0, t1))
            raw["rns_gemm"].append(_us(t1, t2))
            raw["crt_export"].append(_us(t2, t3))
            raw["end_to_end"].append(_us(t0, t3))
    dev = ctx.device_info()
    device = {"device_id": dev.device_id, "name": _text(dev.name), "gcn_arch": _text(dev.gcn_arch),
              "hip_available": 1, "hip_runtime_version": dev.hip_runtime_version,
              "hip_driver_version": dev.hip_driver_version, "global_mem_bytes": dev.global_mem_bytes}
    semantics = "bounded_i64" if signed else "bounded_u64"
    kind = ("per_tile_max_abs" if signed else "per_tile_max_unsigned") if per_tile else (
        "global_max_abs" if signed else "global_max_unsigned")
    rec = build_record(semantics=semantics, bound_kind=kind, bound_mode="per_tile" if per_tile else "global",
                       bound=0 if per_tile else bound, m=m, n=n, k=k, prefix=prefix, tile_m=tm, tile_n=tn,
                       k_block_size=min(k, 65536), tile_bounds=tile_bounds, schedule=schedule,
                       backend=backend_metadata(plan, semantics, m, n, k, prefix, tm, tn), seed=seed,
                       warmups=warmups, repeats=repeats, input_distribution=input_distribution,
                       command_line=command_line, device=device, raw=raw, checksum=checksum_u64(out),
                       git_commit=os.environ.get("RNS8_GIT_COMMIT", "unknown"))
    return rec, out
