"""CPU oracle for rns8 -- TEST INFRASTRUCTURE ONLY.

Loads oracle/liboracle.so (a C restatement of the reference's CPU_REFERENCE
arithmetic, see rns8_oracle.h) and, when it was built in the build container,
oracle/_ref/libref.so (the reference's own header-only reducers compiled in
place). Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
use this module, and only as the checker or the timed CPU baseline; the
product library never calls it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libref.so"

_P = C.c_void_p
_I64 = C.c_int64
_U64 = C.c_uint64
_U32 = C.c_uint32

_PROTOS = {
    "orc_modulus": (C.c_uint16, [_U32]),
    "orc_prefix_range_bits": (C.c_double, [_U32]),
    "orc_ladder_pairwise_coprime": (C.c_int, []),
    "orc_modulus_product": (None, [_U32, _P]),
    "orc_required_prefix_for_range": (_U32, [_P]),
    "orc_select_prefix": (C.c_int, [_U32, _U32, _U64, _I64, _U32, _U32, _U64, _U64, C.POINTER(_U32)]),
    "orc_centered_i64": (C.c_int8, [_I64, _U32]),
    "orc_centered_u64": (C.c_int8, [_U64, _U32]),
    "orc_reduce_to_centered": (C.c_int8, [_I64, _U32]),
    "orc_canonical_from_centered": (_U32, [C.c_int8, _U32]),
    "orc_pack_i64": (None, [_P, _I64, _I64, _I64, _U32, _P]),
    "orc_pack_u64": (None, [_P, _I64, _I64, _I64, _U32, _P]),
    "orc_pack_finite_u8": (None, [_P, _I64, _I64, _I64, _U32, _P]),
    "orc_ring_gemm_modulus": (None, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _U32]),
    "orc_gemm_rns": (None, [_P, _P, _P, _I64, _I64, _I64, _U32]),
    "orc_centered_residue_dot": (C.c_int8, [_P, _P, _I64, _I64, _U32]),
    "orc_reconstruct_canonical": (None, [_P, _U32, _P]),
    "orc_reconstruct_signed": (C.c_int, [_P, _U32, _U64, C.POINTER(_I64)]),
    "orc_reconstruct_unsigned": (C.c_int, [_P, _U32, _U64, C.POINTER(_U64)]),
    "orc_exact_wide_signed_limbs": (C.c_int, [_P, _U32, _P, _U32]),
    "orc_exact_wide_unsigned_limbs": (C.c_int, [_P, _U32, _P, _U32]),
    "orc_export_i64": (C.c_int, [_P, _I64, _I64, _U32, _U64, _P, _I64]),
    "orc_export_u64": (C.c_int, [_P, _I64, _I64, _U32, _U64, _P, _I64]),
    "orc_export_exact_wide_signed": (C.c_int, [_P, _I64, _I64, _U32, _P, _I64, _U32]),
    "orc_export_exact_wide_unsigned": (C.c_int, [_P, _I64, _I64, _U32, _P, _I64, _U32]),
    "orc_export_finite_u8": (None, [_P, _I64, _I64, _U32, _P, _I64]),
    "orc_gemm_i64_rows": (C.c_int, [_P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _U32, _U64, _P, _I64]),
    "orc_gemm_u64_rows": (C.c_int, [_P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _U32, _U64, _P, _I64]),
    "orc_gemm_finite_u8_rows": (None, [_P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _U32, _P, _I64]),
    "orc_gemm_exact_wide_signed_rows": (C.c_int, [_P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _U32, _P, _I64,
                                                  _U32]),
    "orc_exact_gemm_i64": (None, [_P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _U32]),
    "orc_exact_gemm_u64": (None, [_P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _U32]),
    "orc_splitmix64_next": (_U64, [C.POINTER(_U64)]),
    "orc_fill": (None, [_U64, _U32, _U32, _P, _I64]),
    "orc_checksum_u64": (_U64, [_P, _I64, _I64, _I64, _U32]),
    "orc_checksum_u8": (_U64, [_P, _I64, _I64, _I64]),
    "orc_tile_schedule": (C.c_int, [_U32, _I64, _I64, _U32, _U32, _P, _U64, _U32, _U32, _P, _P, _P, _P]),
    "orc_gemm_rns_tiled": (None, [_P, _P, _P, _I64, _I64, _I64, _P, _U64]),
    "orc_export_i64_tiled": (C.c_int, [_P, _I64, _I64, _U32, _U32, _U32, _P, _P, _U64, _P, _I64]),
    "orc_export_u64_tiled": (C.c_int, [_P, _I64, _I64, _U32, _U32, _U32, _P, _P, _U64, _P, _I64]),
    "orc_num_threads": (C.c_int, []),
    "orc_set_num_threads": (None, [C.c_int]),
}



class TileEntry(C.Structure):
    """orc_tile_entry (rns8_oracle.h)."""
    _fields_ = [("flags", _U32), ("tile_row", _U64), ("tile_col", _U64), ("row_offset", _I64),
                ("col_offset", _I64), ("row_extent", _I64), ("col_extent", _I64), ("required_prefix", _U32),
                ("selected_prefix", _U32), ("group_index", _U32), ("range_bit_length", _U32)]


class ScheduleSummary(C.Structure):
    """orc_schedule_summary (rns8_oracle.h)."""
    _fields_ = [("tile_rows", _U64), ("tile_cols", _U64), ("tile_count", _U64), ("min_required", _U32),
                ("max_required", _U32), ("min_selected", _U32), ("max_selected", _U32), ("group_count", _U32),
                ("adaptive_prefix", _U32), ("adaptive_skip", _U32), ("range_bits", _U32), ("flags", _U32),
                ("zero_a_row_count", _U64), ("zero_b_col_count", _U64), ("zero_row_col_product_count", _U64),
                ("collapsed", _U32)]


_lib = None
_ref = None


def build(with_ref: bool = False) -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    if with_ref:
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = C.CDLL(str(LIB))
        for name, (res, args) in _PROTOS.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def ref() -> C.CDLL | None:
    """The reference's own reducers (only where oracle/_ref was built)."""
    global _ref
    if _ref is None and REF_LIB.exists():
        _ref = C.CDLL(str(REF_LIB))
        _ref.ref_reduce_to_centered_i32.restype = C.c_int8
        _ref.ref_reduce_to_centered_i32.argtypes = [C.c_int32, _U32]
        _ref.ref_reduce_to_centered_accelerator_i32.restype = C.c_int8
        _ref.ref_reduce_to_centered_accelerator_i32.argtypes = [C.c_int32, _U32]
        _ref.ref_center_u8.restype = C.c_int8
        _ref.ref_center_u8.argtypes = [C.c_uint8, _U32]
        _ref.ref_canonical_from_centered.restype = _U32
        _ref.ref_canonical_from_centered.argtypes = [C.c_int8, _U32]
        _ref.ref_centered_residue_dot.restype = C.c_int8
        _ref.ref_centered_residue_dot.argtypes = [_P, _P, _I64, _I64, _U32]
        _ref.ref_reduce_many.restype = None
        _ref.ref_reduce_many.argtypes = [_P, _I64, _U32, _P]
    return _ref


def _p(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


LADDER = [256, 255, 253, 251, 247, 239, 233, 229, 227, 223, 217, 211, 199, 197, 193, 191, 181, 179, 173, 167, 163,
          157, 151, 149, 139, 137, 131, 127]


def modulus_product(prefix: int) -> int:
    out = np.zeros(4, dtype=np.uint64)
    lib().orc_modulus_product(prefix, _p(out))
    return sum(int(w) << (64 * i) for i, w in enumerate(out))


def pack_i64(src: np.ndarray, prefix: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.int64)
    rows, cols = src.shape
    out = np.empty((prefix, rows, cols), dtype=np.int8)
    lib().orc_pack_i64(_p(src), rows, cols, cols, prefix, _p(out))
    return out


def pack_u64(src: np.ndarray, prefix: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint64)
    rows, cols = src.shape
    out = np.empty((prefix, rows, cols), dtype=np.int8)
    lib().orc_pack_u64(_p(src), rows, cols, cols, prefix, _p(out))
    return out


def pack_finite_u8(src: np.ndarray, modulus: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    rows, cols = src.shape
    out = np.empty((rows, cols), dtype=np.int8)
    lib().orc_pack_finite_u8(_p(src), rows, cols, cols, modulus, _p(out))
    return out


def ring_gemm(A: np.ndarray, B: np.ndarray, modulus: int) -> np.ndarray:
    A = np.ascontiguousarray(A, dtype=np.int8)
    B = np.ascontiguousarray(B, dtype=np.int8)
    m, k = A.shape
    n = B.shape[1]
    out = np.empty((m, n), dtype=np.int8)
    lib().orc_ring_gemm_modulus(_p(A), _p(B), _p(out), m, n, k, k, n, n, modulus)
    return out


def gemm_rns(Ap: np.ndarray, Bp: np.ndarray, prefix: int) -> np.ndarray:
    Ap = np.ascontiguousarray(Ap[:prefix], dtype=np.int8)
    Bp = np.ascontiguousarray(Bp[:prefix], dtype=np.int8)
    _, m, k = Ap.shape
    n = Bp.shape[2]
    out = np.empty((prefix, m, n), dtype=np.int8)
    lib().orc_gemm_rns(_p(Ap), _p(Bp), _p(out), m, n, k, prefix)
    return out


def export_i64(Cp: np.ndarray, prefix: int, bound: int):
    Cp = np.ascontiguousarray(Cp[:prefix], dtype=np.int8)
    _, m, n = Cp.shape
    out = np.zeros((m, n), dtype=np.int64)
    st = lib().orc_export_i64(_p(Cp), m, n, prefix, bound, _p(out), n)
    return st, out


def export_u64(Cp: np.ndarray, prefix: int, bound: int):
    Cp = np.ascontiguousarray(Cp[:prefix], dtype=np.int8)
    _, m, n = Cp.shape
    out = np.zeros((m, n), dtype=np.uint64)
    st = lib().orc_export_u64(_p(Cp), m, n, prefix, bound, _p(out), n)
    return st, out


def export_exact_wide(Cp: np.ndarray, prefix: int, limbs: int, signed: bool):
    Cp = np.ascontiguousarray(Cp[:prefix], dtype=np.int8)
    _, m, n = Cp.shape
    out = np.zeros((m, n * limbs), dtype=np.uint64)
    fn = lib().orc_export_exact_wide_signed if signed else lib().orc_export_exact_wide_unsigned
    st = fn(_p(Cp), m, n, prefix, _p(out), n, limbs)
    return st, out


def export_finite_u8(Cp: np.ndarray, modulus: int) -> np.ndarray:
    Cp = np.ascontiguousarray(Cp, dtype=np.int8)
    m, n = Cp.shape
    out = np.zeros((m, n), dtype=np.uint8)
    lib().orc_export_finite_u8(_p(Cp), m, n, modulus, _p(out), n)
    return out


def gemm_i64(A: np.ndarray, B: np.ndarray, prefix: int, bound: int, row0: int = 0, rows: int | None = None):
    """CPU_REFERENCE pipeline (pack -> ring GEMM -> export) for rows [row0, row0+rows)."""
    A = np.ascontiguousarray(A, dtype=np.int64)
    B = np.ascontiguousarray(B, dtype=np.int64)
    m, k = A.shape
    n = B.shape[1]
    rows = m - row0 if rows is None else rows
    out = np.zeros((rows, n), dtype=np.int64)
    st = lib().orc_gemm_i64_rows(_p(A), k, _p(B), n, k, n, row0, rows, prefix, bound, _p(out), n)
    return st, out


def gemm_u64(A: np.ndarray, B: np.ndarray, prefix: int, bound: int, row0: int = 0, rows: int | None = None):
    A = np.ascontiguousarray(A, dtype=np.uint64)
    B = np.ascontiguousarray(B, dtype=np.uint64)
    m, k = A.shape
    n = B.shape[1]
    rows = m - row0 if rows is None else rows
    out = np.zeros((rows, n), dtype=np.uint64)
    st = lib().orc_gemm_u64_rows(_p(A), k, _p(B), n, k, n, row0, rows, prefix, bound, _p(out), n)
    return st, out


def gemm_finite_u8(A: np.ndarray, B: np.ndarray, modulus: int, row0: int = 0, rows: int | None = None):
    A = np.ascontiguousarray(A, dtype=np.uint8)
    B = np.ascontiguousarray(B, dtype=np.uint8)
    m, k = A.shape
    n = B.shape[1]
    rows = m - row0 if rows is None else rows
    out = np.zeros((rows, n), dtype=np.uint8)
    lib().orc_gemm_finite_u8_rows(_p(A), k, _p(B), n, k, n, row0, rows, modulus, _p(out), n)
    return out


def gemm_exact_wide_signed(A: np.ndarray, B: np.ndarray, prefix: int, limbs: int, row0: int = 0,
                           rows: int | None = None):
    A = np.ascontiguousarray(A, dtype=np.int64)
    B = np.ascontiguousarray(B, dtype=np.int64)
    m, k = A.shape
    n = B.shape[1]
    rows = m - row0 if rows is None else rows
    out = np.zeros((rows, n * limbs), dtype=np.uint64)
    st = lib().orc_gemm_exact_wide_signed_rows(_p(A), k, _p(B), n, k, n, row0, rows, prefix, _p(out), n, limbs)
    return st, out


def exact_gemm_i64(A: np.ndarray, B: np.ndarray, limbs: int = 4) -> np.ndarray:
    """Brute-force sum of int64 products in two's complement limbs (no RNS)."""
    A = np.ascontiguousarray(A, dtype=np.int64)
    B = np.ascontiguousarray(B, dtype=np.int64)
    m, k = A.shape
    n = B.shape[1]
    out = np.zeros((m, n * limbs), dtype=np.uint64)
    lib().orc_exact_gemm_i64(_p(A), k, _p(B), n, m, n, k, _p(out), n, limbs)
    return out


def exact_gemm_u64(A: np.ndarray, B: np.ndarray, limbs: int = 4) -> np.ndarray:
    A = np.ascontiguousarray(A, dtype=np.uint64)
    B = np.ascontiguousarray(B, dtype=np.uint64)
    m, k = A.shape
    n = B.shape[1]
    out = np.zeros((m, n * limbs), dtype=np.uint64)
    lib().orc_exact_gemm_u64(_p(A), k, _p(B), n, m, n, k, _p(out), n, limbs)
    return out


def limbs_to_int(row: np.ndarray, signed: bool) -> int:
    v = sum(int(w) << (64 * i) for i, w in enumerate(row))
    bits = 64 * len(row)
    if signed and v >> (bits - 1):
        v -= 1 << bits
    return v


def fill(seed: int, mode: int, param: int, count: int, dtype) -> np.ndarray:
    out = np.empty(count, dtype=dtype)
    lib().orc_fill(seed, mode, param, _p(out), count)
    return out


def checksum_u64(values: np.ndarray, limbs: int = 1) -> int:
    v = np.ascontiguousarray(values).view(np.uint64)
    rows = v.shape[0]
    cols = v.shape[1] // limbs
    return int(lib().orc_checksum_u64(_p(v), rows, cols, cols, limbs))


def set_threads(n: int) -> None:
    lib().orc_set_num_threads(n)


def threads() -> int:
    return int(lib().orc_num_threads())


SEM_BOUNDED_I64, SEM_BOUNDED_U64 = 1, 2


def tile_schedule(signed: bool, m: int, n: int, tile_m: int, tile_n: int, bounds, budget: int, flags: int = 0,
                  zero_a_rows=None, zero_b_cols=None):
    """Per-tile bounded schedule: (status, entries, summary) as ctypes records."""
    b = np.ascontiguousarray(np.asarray(bounds, dtype=np.uint64))
    tm = tile_m or 128
    tn = tile_n or 128
    count = ((m + tm - 1) // tm) * ((n + tn - 1) // tn)
    entries = (TileEntry * max(count, 1))()
    summary = ScheduleSummary()
    za = None if zero_a_rows is None else np.ascontiguousarray(zero_a_rows, dtype=np.uint8)
    zb = None if zero_b_cols is None else np.ascontiguousarray(zero_b_cols, dtype=np.uint8)
    st = lib().orc_tile_schedule(SEM_BOUNDED_I64 if signed else SEM_BOUNDED_U64, m, n, tile_m, tile_n, _p(b), len(b),
                                 budget, flags, None if za is None else _p(za), None if zb is None else _p(zb),
                                 C.cast(entries, C.c_void_p), C.byref(summary))
    return st, list(entries)[:count], summary


def _entry_array(entries):
    arr = (TileEntry * max(len(entries), 1))()
    for i, e in enumerate(entries):
        arr[i] = e
    return arr


def gemm_rns_tiled(Ap: np.ndarray, Bp: np.ndarray, Cp: np.ndarray, entries) -> np.ndarray:
    """Tiled plane GEMM into a copy of Cp (planes beyond a tile's prefix keep Cp's values)."""
    Ap = np.ascontiguousarray(Ap, dtype=np.int8)
    Bp = np.ascontiguousarray(Bp, dtype=np.int8)
    out = np.array(Cp, dtype=np.int8, order="C", copy=True)
    _, m, k = Ap.shape
    n = Bp.shape[2]
    arr = _entry_array(entries)
    lib().orc_gemm_rns_tiled(_p(Ap), _p(Bp), _p(out), m, n, k, C.cast(arr, C.c_void_p), len(entries))
    return out


def export_tiled(Cp: np.ndarray, tile_m: int, tile_n: int, entries, bounds, signed: bool):
    Cp = np.ascontiguousarray(Cp, dtype=np.int8)
    P, m, n = Cp.shape
    b = np.ascontiguousarray(np.asarray(bounds, dtype=np.uint64))
    arr = _entry_array(entries)
    out = np.zeros((m, n), dtype=np.int64 if signed else np.uint64)
    fn = lib().orc_export_i64_tiled if signed else lib().orc_export_u64_tiled
    st = fn(_p(Cp), m, n, P, tile_m or 128, tile_n or 128, C.cast(arr, C.c_void_p), _p(b), len(entries), _p(out), n)
    return st, out
