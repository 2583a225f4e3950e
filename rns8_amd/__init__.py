"""rns8 for MI355X: Python host mirror of the rns8 C ABI.

The product is the shared library rns8_amd/librns8.so (C ABI in include/,
gfx950 kernels in rns8_amd/csrc/). This module binds it through ctypes with
the same entry-point names, argument meaning and status codes, so tests and
the benchmark drive exactly what a C caller would. There is no fallback: if
the library is missing, `lib()` raises.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import abi
from .abi import (  # noqa: F401  (re-exported constants)
    BACKEND_AUTO,
    BACKEND_CPU_REFERENCE,
    BACKEND_HIP_DIRECT,
    BOUND_GLOBAL_MAX_ABS,
    BOUND_GLOBAL_MAX_UNSIGNED,
    BOUND_INPUT_RANGE_AND_K,
    BOUND_NONE,
    BOUND_PER_TILE_MAX_ABS,
    BOUND_PER_TILE_MAX_UNSIGNED,
    BOUNDED_I64,
    BOUNDED_U64,
    EXACT_AXES_CARRIED,
    EXACT_AXES_NATIVE,
    EXACT_AXES_NONE,
    EXACT_WIDE_SIGNED,
    EXACT_WIDE_UNSIGNED,
    FINITE_FIELD_U8,
    FINITE_RING_U8,
    INVALID_ARGUMENT,
    PLAN_ALLOW_PROVEN_ZERO_TILE_SKIPS,
    PLAN_FORCE_FIXED_PREFIX,
    RANGE_ERROR,
    SUCCESS,
    UNSUPPORTED_BACKEND,
)

_LIB = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = abi.load_library()
    return _LIB


class Rns8Error(RuntimeError):
    def __init__(self, what: str, status: int):
        super().__init__(f"{what}: {status_string(status)} ({status})")
        self.status = status


def status_string(status: int) -> str:
    return lib().rns8_status_string(status).decode()


def check(status: int, what: str) -> None:
    if status != abi.SUCCESS:
        raise Rns8Error(what, status)


def gemm_desc(semantics, bound_kind, m, n, k, bound=0, max_prefix=0, flags=0, finite_modulus=0, lhs_bound=0,
              rhs_bound=0, requested_backend=BACKEND_AUTO, tile_m=0, tile_n=0, tile_bounds=None, zero_a_rows=None,
              zero_b_cols=None) -> abi.GemmDesc:
    """A gemm descriptor; per-tile bounds and zero proof masks are kept alive on
    the returned object (the library copies them at plan creation)."""
    d = abi.new_struct(abi.GemmDesc)
    if tile_bounds is not None:
        d._tile_bounds = (C.c_uint64 * max(len(tile_bounds), 1))(*[int(b) for b in tile_bounds])
        d.tile_bounds = C.cast(d._tile_bounds, C.POINTER(C.c_uint64))
        d.tile_bounds_count = len(tile_bounds)
    if zero_a_rows is not None:
        d._zero_a = (C.c_uint8 * max(len(zero_a_rows), 1))(*[int(v) for v in zero_a_rows])
        d.zero_a_rows = C.cast(d._zero_a, C.POINTER(C.c_uint8))
        d.zero_a_rows_count = len(zero_a_rows)
    if zero_b_cols is not None:
        d._zero_b = (C.c_uint8 * max(len(zero_b_cols), 1))(*[int(v) for v in zero_b_cols])
        d.zero_b_cols = C.cast(d._zero_b, C.POINTER(C.c_uint8))
        d.zero_b_cols_count = len(zero_b_cols)
    d.semantics = semantics
    d.bound_kind = bound_kind
    d.requested_backend = requested_backend
    d.m, d.n, d.k = m, n, k
    d.bound = bound
    d.max_prefix = max_prefix
    d.tile_m, d.tile_n = tile_m, tile_n
    d.finite_modulus = finite_modulus
    d.flags = flags
    d.lhs_bound, d.rhs_bound = lhs_bound, rhs_bound
    return d


def matrix_desc(rows, cols, semantics, bound_kind, max_prefix=0, logical_ld=0, tile_m=0, tile_n=0) -> abi.MatrixDesc:
    d = abi.new_struct(abi.MatrixDesc)
    d.rows, d.cols = rows, cols
    d.logical_ld = logical_ld
    d.semantics = semantics
    d.logical_layout = abi.LAYOUT_ROW_MAJOR
    d.bound_kind = bound_kind
    d.tile_m, d.tile_n = tile_m, tile_n
    d.max_prefix = max_prefix
    return d


def select_prefix(desc: abi.GemmDesc) -> tuple[int, int]:
    """(status, prefix) for the plan `desc` would create (no device needed)."""
    out = C.c_uint32(0)
    st = lib().rns8_mi355x_select_prefix(C.byref(desc), C.byref(out))
    return st, out.value


def plan_schedule(desc: abi.GemmDesc):
    """(status, info, entries) of the schedule a plan from `desc` would build (no device needed)."""
    info = abi.new_struct(abi.PlanScheduleInfo)
    written = C.c_uint64(0)
    st = lib().rns8_mi355x_plan_schedule(C.byref(desc), C.byref(info), None, 0, C.byref(written))
    if st != abi.SUCCESS:
        return st, None, []
    entries = (abi.TileScheduleEntry * max(written.value, 1))()
    for e in entries:
        e.struct_size = C.sizeof(abi.TileScheduleEntry)
        e.abi_version = abi.ABI_VERSION
    st = lib().rns8_mi355x_plan_schedule(C.byref(desc), C.byref(info), C.cast(entries, C.c_void_p), written.value,
                                         C.byref(written))
    return st, info, list(entries)[:written.value]


def _ptr(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


class _Handle:
    _destroy = ""

    def __init__(self):
        self.ptr = C.c_void_p()

    def close(self):
        if self.ptr:
            getattr(lib(), self._destroy)(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Context(_Handle):
    _destroy = "rns8_destroy_context"

    def __init__(self, device_id: int = -1, backend: int | None = None):
        super().__init__()
        opts = None
        if backend is not None:
            opts = abi.new_struct(abi.ContextOptions)
            opts.requested_backend = backend
        st = lib().rns8_create_context(device_id, C.byref(opts) if opts is not None else None, C.byref(self.ptr))
        check(st, "rns8_create_context")

    def device_info(self) -> abi.DeviceInfo:
        info = abi.new_struct(abi.DeviceInfo)
        check(lib().rns8_get_device_info(self.ptr, C.byref(info)), "rns8_get_device_info")
        return info


class Plan(_Handle):
    _destroy = "rns8_destroy_plan"

    def __init__(self, ctx: Context, desc: abi.GemmDesc):
        super().__init__()
        self.desc = desc
        check(lib().rns8_create_plan(ctx.ptr, C.byref(desc), C.byref(self.ptr)), "rns8_create_plan")

    def schedule_info(self) -> abi.PlanScheduleInfo:
        info = abi.new_struct(abi.PlanScheduleInfo)
        check(lib().rns8_get_plan_schedule_info(self.ptr, C.byref(info)), "rns8_get_plan_schedule_info")
        return info

    def tile_schedule(self) -> list:
        written = C.c_uint64(0)
        check(lib().rns8_get_plan_tile_schedule(self.ptr, None, 0, C.byref(written)), "rns8_get_plan_tile_schedule")
        entries = (abi.TileScheduleEntry * max(written.value, 1))()
        check(lib().rns8_get_plan_tile_schedule(self.ptr, C.cast(entries, C.c_void_p), written.value,
                                                C.byref(written)), "rns8_get_plan_tile_schedule")
        return list(entries)[:written.value]

    @property
    def prefix(self) -> int:
        return self.schedule_info().max_selected_prefix

    def backend_info(self) -> abi.PlanBackendInfo:
        info = abi.new_struct(abi.PlanBackendInfo)
        check(lib().rns8_get_plan_backend_info(self.ptr, C.byref(info)), "rns8_get_plan_backend_info")
        return info

    def selected_kernel(self) -> str:
        """The kernel the plan's GEMM runs, as rns8_get_plan_backend_info names it."""
        return bytes(self.backend_info().selected_kernel).split(b"\0", 1)[0].decode()


class Workspace(_Handle):
    _destroy = "rns8_destroy_workspace"

    def __init__(self, ctx: Context, plan: Plan):
        super().__init__()
        check(lib().rns8_create_workspace(ctx.ptr, plan.ptr, C.byref(self.ptr)), "rns8_create_workspace")


class Matrix(_Handle):
    _destroy = "rns8_destroy_matrix"

    def __init__(self, ctx: Context, desc: abi.MatrixDesc):
        super().__init__()
        self.rows, self.cols = desc.rows, desc.cols
        check(lib().rns8_create_matrix(ctx.ptr, C.byref(desc), C.byref(self.ptr)), "rns8_create_matrix")

    def storage_info(self) -> abi.MatrixStorageInfo:
        info = abi.new_struct(abi.MatrixStorageInfo)
        check(lib().rns8_get_matrix_storage_info(self.ptr, C.byref(info)), "rns8_get_matrix_storage_info")
        return info

    def planes(self):
        p, rp, pp, n = C.c_void_p(), C.c_int64(), C.c_int64(), C.c_uint32()
        check(lib().rns8_mi355x_get_matrix_planes(self.ptr, C.byref(p), C.byref(rp), C.byref(pp), C.byref(n)),
              "rns8_mi355x_get_matrix_planes")
        return p.value, rp.value, pp.value, n.value

    def exact_proof(self, ctx: Context):
        """The exact-wide magnitude proof this matrix carries
        (rns8_mi355x_get_exact_proof): (bound, kind, rows, cols), with rows
        and cols lists of dicts of Python integers (max_magnitude,
        absolute_sum, sum, minimum, maximum, deviation_sum) and kind one of
        EXACT_AXES_NATIVE / EXACT_AXES_CARRIED / EXACT_AXES_NONE."""
        bound = np.zeros(4, dtype=np.uint64)
        kind = C.c_uint32()
        rows = np.zeros((self.rows, 16), dtype=np.uint64)
        cols = np.zeros((self.cols, 16), dtype=np.uint64)
        check(lib().rns8_mi355x_get_exact_proof(ctx.ptr, self.ptr, bound.ctypes.data, C.byref(kind),
                                                rows.ctypes.data, cols.ctypes.data), "rns8_mi355x_get_exact_proof")

        def word_int(w, signed=False):
            v = sum(int(x) << (64 * i) for i, x in enumerate(w))
            bits = 64 * len(w)
            return v - (1 << bits) if signed and v >> (bits - 1) else v

        def axis(r):
            return {"max_magnitude": word_int(r[0:4]), "absolute_sum": word_int(r[4:8]),
                    "sum": word_int(r[8:10], True), "minimum": word_int(r[10:12], True),
                    "maximum": word_int(r[12:14], True), "deviation_sum": word_int(r[14:16])}

        k = kind.value
        if k == EXACT_AXES_NONE:
            return word_int(bound), k, [], []
        return word_int(bound), k, [axis(r) for r in rows], [axis(c) for c in cols]

    def read_residues(self, nplanes: int | None = None) -> np.ndarray:
        """Copy the resident planes to host as int8 [planes][rows][cols]."""
        from . import hip

        ptr, row_pitch, plane_pitch, count = self.planes()
        count = count if nplanes is None else nplanes
        raw = np.empty(plane_pitch * count, dtype=np.int8)
        hip.from_device(raw, ptr)
        out = np.empty((count, self.rows, self.cols), dtype=np.int8)
        for p in range(count):
            plane = raw[p * plane_pitch:p * plane_pitch + self.rows * row_pitch].reshape(self.rows, row_pitch)
            out[p] = plane[:, :self.cols]
        return out


# ---- host entry points (status-returning, like the C ABI) -------------------


def pack_i64(ctx, matrix, src: np.ndarray, source_version=0, ld=None) -> int:
    src = np.ascontiguousarray(src, dtype=np.int64) if ld is None else src
    return lib().rns8_pack_i64(ctx.ptr, matrix.ptr, _ptr(src), ld or src.shape[1], source_version)


def pack_u64(ctx, matrix, src: np.ndarray, source_version=0, ld=None) -> int:
    src = np.ascontiguousarray(src, dtype=np.uint64) if ld is None else src
    return lib().rns8_pack_u64(ctx.ptr, matrix.ptr, _ptr(src), ld or src.shape[1], source_version)


def pack_finite_u8(ctx, matrix, modulus, src: np.ndarray, source_version=0, ld=None) -> int:
    src = np.ascontiguousarray(src, dtype=np.uint8) if ld is None else src
    return lib().rns8_pack_finite_u8(ctx.ptr, matrix.ptr, modulus, _ptr(src), ld or src.shape[1], source_version)


def gemm_rns(ctx, plan, A, B, Cm, ws) -> int:
    return lib().rns8_gemm_rns(ctx.ptr, plan.ptr, A.ptr, B.ptr, Cm.ptr, ws.ptr)


def gemm_finite_u8(ctx, plan, modulus, A, B, Cm, ws) -> int:
    return lib().rns8_gemm_finite_u8(ctx.ptr, plan.ptr, modulus, A.ptr, B.ptr, Cm.ptr, ws.ptr)


def grouped_tasks(triplets):
    """ctypes array of rns8_grouped_gemm_task from (A, B, C, workspace) handle tuples."""
    arr = (abi.GroupedGemmTask * max(len(triplets), 1))()
    for i, (a, b, c, w) in enumerate(triplets):
        arr[i].struct_size = C.sizeof(abi.GroupedGemmTask)
        arr[i].abi_version = abi.ABI_VERSION
        arr[i].a, arr[i].b, arr[i].c, arr[i].workspace = a.ptr, b.ptr, c.ptr, w.ptr
    return arr


def gemm_rns_grouped(ctx, plan, triplets, tasks=None) -> int:
    tasks = grouped_tasks(triplets) if tasks is None else tasks
    return lib().rns8_gemm_rns_grouped(ctx.ptr, plan.ptr, tasks, len(triplets))


def gemm_finite_u8_grouped(ctx, plan, modulus, triplets) -> int:
    return lib().rns8_gemm_finite_u8_grouped(ctx.ptr, plan.ptr, modulus, grouped_tasks(triplets), len(triplets))


def grouped_contract_info(plan, task_count) -> tuple[int, abi.GroupedDispatchContractInfo]:
    info = abi.new_struct(abi.GroupedDispatchContractInfo)
    st = lib().rns8_get_grouped_dispatch_contract_info(plan.ptr, task_count, C.byref(info))
    return st, info


def export_i64(ctx, plan, Cm, dst: np.ndarray) -> int:
    return lib().rns8_export_i64(ctx.ptr, plan.ptr, Cm.ptr, _ptr(dst), dst.shape[1])


def export_u64(ctx, plan, Cm, dst: np.ndarray) -> int:
    return lib().rns8_export_u64(ctx.ptr, plan.ptr, Cm.ptr, _ptr(dst), dst.shape[1])


def export_finite_u8(ctx, plan, modulus, Cm, dst: np.ndarray) -> int:
    return lib().rns8_export_finite_u8(ctx.ptr, plan.ptr, modulus, Cm.ptr, _ptr(dst), dst.shape[1])


def export_exact_wide_signed_limbs(ctx, plan, Cm, dst: np.ndarray, limbs: int) -> int:
    """dst: uint64 [rows][ld*limbs] (element (r, c) at dst[r, c*limbs:(c+1)*limbs])."""
    return lib().rns8_export_exact_wide_signed_limbs(ctx.ptr, plan.ptr, Cm.ptr, _ptr(dst), dst.shape[1] // limbs, limbs)


def export_exact_wide_unsigned_limbs(ctx, plan, Cm, dst: np.ndarray, limbs: int) -> int:
    return lib().rns8_export_exact_wide_unsigned_limbs(ctx.ptr, plan.ptr, Cm.ptr, _ptr(dst), dst.shape[1] // limbs,
                                                       limbs)


def gemm_i64_oneshot(ctx, desc, A: np.ndarray, B: np.ndarray, C_out: np.ndarray | None = None):
    A = np.ascontiguousarray(A, dtype=np.int64)
    B = np.ascontiguousarray(B, dtype=np.int64)
    out = C_out if C_out is not None else np.zeros((A.shape[0], B.shape[1]), dtype=np.int64)
    st = lib().rns8_gemm_i64_oneshot(ctx.ptr, C.byref(desc), _ptr(A), A.shape[1], _ptr(B), B.shape[1], _ptr(out),
                                     out.shape[1])
    return st, out


def gemm_u64_oneshot(ctx, desc, A: np.ndarray, B: np.ndarray, C_out: np.ndarray | None = None):
    A = np.ascontiguousarray(A, dtype=np.uint64)
    B = np.ascontiguousarray(B, dtype=np.uint64)
    out = C_out if C_out is not None else np.zeros((A.shape[0], B.shape[1]), dtype=np.uint64)
    st = lib().rns8_gemm_u64_oneshot(ctx.ptr, C.byref(desc), _ptr(A), A.shape[1], _ptr(B), B.shape[1], _ptr(out),
                                     out.shape[1])
    return st, out


def gemm_finite_u8_oneshot(ctx, desc, modulus, A: np.ndarray, B: np.ndarray, field: bool,
                           C_out: np.ndarray | None = None):
    A = np.ascontiguousarray(A, dtype=np.uint8)
    B = np.ascontiguousarray(B, dtype=np.uint8)
    out = C_out if C_out is not None else np.zeros((A.shape[0], B.shape[1]), dtype=np.uint8)
    fn = lib().rns8_gemm_finite_field_u8_oneshot if field else lib().rns8_gemm_finite_ring_u8_oneshot
    st = fn(ctx.ptr, C.byref(desc), modulus, _ptr(A), A.shape[1], _ptr(B), B.shape[1], _ptr(out), out.shape[1])
    return st, out
