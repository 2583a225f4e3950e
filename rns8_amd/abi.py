"""ctypes mirror of the rns8 C ABI (include/rns8/rns8.h, include/rns8_mi355x.h).

Struct layouts, enum values and signatures follow the headers one to one so
Python tests and the benchmark call the shared library exactly as a C caller
would. Only the structs the hot path needs are mirrored field by field.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

ABI_VERSION = 1

# rns8_status (status.h)
SUCCESS = 0
INVALID_ARGUMENT = 1
UNSUPPORTED_OS = 2
UNSUPPORTED_ARCH = 3
UNSUPPORTED_BACKEND = 4
RANGE_ERROR = 5
ACCUMULATION_OVERFLOW_RISK = 6
WORKSPACE_TOO_SMALL = 7
BACKEND_FAILURE = 8
VERIFICATION_FAILED = 9
INTERNAL_ERROR = 10

# rns8_semantics (semantics.h)
BOUNDED_I64 = 1
BOUNDED_U64 = 2
EXACT_WIDE_SIGNED = 3
EXACT_WIDE_UNSIGNED = 4
WRAP_U64_MOD_2_64 = 5
FINITE_RING_U8 = 6
FINITE_FIELD_U8 = 7

# rns8_layout
LAYOUT_ROW_MAJOR = 1
LAYOUT_COLUMN_MAJOR = 2

# rns8_backend_kind
BACKEND_AUTO = 0
BACKEND_CPU_REFERENCE = 1
BACKEND_HIP_DIRECT = 2

# rns8_bound_kind (bounds.h)
BOUND_NONE = 0
BOUND_GLOBAL_MAX_ABS = 1
BOUND_GLOBAL_MAX_UNSIGNED = 2
BOUND_PER_TILE_MAX_ABS = 3
BOUND_PER_TILE_MAX_UNSIGNED = 4
BOUND_INPUT_RANGE_AND_K = 5

# plan flags
PLAN_FORCE_FIXED_PREFIX = 0x1
PLAN_ALLOW_PROVEN_ZERO_TILE_SKIPS = 0x2
PLAN_ALLOW_PROVEN_ZERO_ROW_COL_SKIPS = 0x4

# rns8_mi355x_get_exact_proof axis kinds
EXACT_AXES_NATIVE = 0
EXACT_AXES_CARRIED = 1
EXACT_AXES_NONE = 2

DEFAULT_MODULUS_COUNT = 28
DEFAULT_BOUNDED_PREFIX = 9
MAX_SUPPORTED_PREFIX = 20
SAFE_INT32_K_BLOCK = 65536


class ContextOptions(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint64),
        ("abi_version", C.c_uint32),
        ("requested_backend", C.c_uint32),
        ("flags", C.c_uint32),
    ]


class DeviceInfo(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint64),
        ("abi_version", C.c_uint32),
        ("backend", C.c_uint32),
        ("device_id", C.c_int32),
        ("hip_available", C.c_uint32),
        ("hip_runtime_version", C.c_uint32),
        ("hip_driver_version", C.c_uint32),
        ("global_mem_bytes", C.c_uint64),
        ("name", C.c_char * 128),
        ("gcn_arch", C.c_char * 64),
        ("detail", C.c_char * 256),
    ]


class GemmDesc(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint64),
        ("abi_version", C.c_uint32),
        ("semantics", C.c_uint32),
        ("bound_kind", C.c_uint32),
        ("requested_backend", C.c_uint32),
        ("m", C.c_int64),
        ("n", C.c_int64),
        ("k", C.c_int64),
        ("bound", C.c_uint64),
        ("max_prefix", C.c_uint32),
        ("tile_m", C.c_uint32),
        ("tile_n", C.c_uint32),
        ("finite_modulus", C.c_uint32),
        ("flags", C.c_uint32),
        ("tile_bounds", C.POINTER(C.c_uint64)),
        ("tile_bounds_count", C.c_uint64),
        ("lhs_bound", C.c_uint64),
        ("rhs_bound", C.c_uint64),
        ("zero_a_rows", C.POINTER(C.c_uint8)),
        ("zero_a_rows_count", C.c_uint64),
        ("zero_b_cols", C.POINTER(C.c_uint8)),
        ("zero_b_cols_count", C.c_uint64),
    ]


class MatrixDesc(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint64),
        ("abi_version", C.c_uint32),
        ("rows", C.c_int64),
        ("cols", C.c_int64),
        ("logical_ld", C.c_int64),
        ("semantics", C.c_uint32),
        ("logical_layout", C.c_uint32),
        ("bound_kind", C.c_uint32),
        ("tile_m", C.c_uint32),
        ("tile_n", C.c_uint32),
        ("max_prefix", C.c_uint32),
        ("flags", C.c_uint32),
    ]


class PlanScheduleInfo(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint64),
        ("abi_version", C.c_uint32),
        ("tile_m", C.c_uint32),
        ("tile_n", C.c_uint32),
        ("tile_rows", C.c_uint64),
        ("tile_cols", C.c_uint64),
        ("tile_count", C.c_uint64),
        ("min_required_prefix", C.c_uint32),
        ("max_required_prefix", C.c_uint32),
        ("min_selected_prefix", C.c_uint32),
        ("max_selected_prefix", C.c_uint32),
        ("prefix_group_count", C.c_uint32),
        ("adaptive_prefix_active", C.c_uint32),
        ("adaptive_skip_active", C.c_uint32),
        ("range_bit_length", C.c_uint32),
        ("flags", C.c_uint32),
        ("bound_kind", C.c_uint32),
        ("reserved0", C.c_uint32),
        ("effective_bound", C.c_uint64),
        ("lhs_bound", C.c_uint64),
        ("rhs_bound", C.c_uint64),
        ("zero_a_row_count", C.c_uint64),
        ("zero_b_col_count", C.c_uint64),
        ("zero_row_col_product_count", C.c_uint64),
        ("bound_contract", C.c_char * 96),
    ]


class TileScheduleEntry(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint64),
        ("abi_version", C.c_uint32),
        ("flags", C.c_uint32),
        ("tile_row", C.c_uint64),
        ("tile_col", C.c_uint64),
        ("row_offset", C.c_int64),
        ("col_offset", C.c_int64),
        ("row_extent", C.c_int64),
        ("col_extent", C.c_int64),
        ("required_prefix", C.c_uint32),
        ("selected_prefix", C.c_uint32),
        ("group_index", C.c_uint32),
        ("range_bit_length", C.c_uint32),
    ]


class MatrixStorageInfo(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint64),
        ("abi_version", C.c_uint32),
        ("backend", C.c_uint32),
        ("semantics", C.c_uint32),
        ("logical_layout", C.c_uint32),
        ("bound_kind", C.c_uint32),
        ("rows", C.c_int64),
        ("cols", C.c_int64),
        ("logical_ld", C.c_int64),
        ("max_prefix", C.c_uint32),
        ("finite_modulus", C.c_uint32),
        ("matrix_instance_id", C.c_uint64),
        ("source_version", C.c_uint64),
        ("host_residues_current", C.c_uint32),
        ("device_residues_current", C.c_uint32),
        ("host_byte_limbs_current", C.c_uint32),
        ("device_byte_limbs_current", C.c_uint32),
        ("host_native_current", C.c_uint32),
        ("device_native_current", C.c_uint32),
        ("uses_residue_storage", C.c_uint32),
        ("uses_byte_limb_storage", C.c_uint32),
        ("uses_native_storage", C.c_uint32),
        ("hip_device_id", C.c_int32),
        ("flags", C.c_uint32),
        ("host_residue_bytes", C.c_uint64),
        ("device_residue_bytes", C.c_uint64),
        ("host_byte_limb_bytes", C.c_uint64),
        ("device_byte_limb_bytes", C.c_uint64),
        ("host_native_bytes", C.c_uint64),
        ("device_native_bytes", C.c_uint64),
        ("layout_version", C.c_char * 96),
        ("storage_scope", C.c_char * 96),
        ("detail", C.c_char * 256),
    ]


class PlanBackendInfo(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint64),
        ("abi_version", C.c_uint32),
        ("backend", C.c_uint32),
        ("is_accelerator", C.c_uint32),
        ("is_correctness_backend", C.c_uint32),
        ("is_matrix_engine_backend", C.c_uint32),
        ("compiled_kernel_available", C.c_uint32),
        ("exact_differential_validated", C.c_uint32),
        ("performance_validated", C.c_uint32),
        ("flags", C.c_uint32),
        ("workspace_required_bytes", C.c_uint64),
        ("selected_kernel", C.c_char * 128),
        ("accelerator_library", C.c_char * 64),
        ("accelerator_version", C.c_char * 64),
        ("capability_status", C.c_char * 128),
        ("epilogue_mode", C.c_char * 96),
        ("workspace_mode", C.c_char * 96),
        ("isa_evidence", C.c_char * 128),
        ("autotune_key", C.c_char * 1024),
        ("accumulator_k_block_size", C.c_uint64),
        ("accumulator_k_block_cap", C.c_uint64),
        ("accumulator_modulus", C.c_uint64),
        ("accumulator_max_lhs_abs", C.c_uint64),
        ("accumulator_max_rhs_abs", C.c_uint64),
        ("accumulator_max_product", C.c_uint64),
        ("accumulator_uses_int32_inner_product", C.c_uint32),
        ("accumulator_safe_for_k_block", C.c_uint32),
        ("accumulator_input_domain", C.c_char * 64),
        ("accumulator_signedness", C.c_char * 64),
        ("accumulator_type", C.c_char * 64),
        ("accumulator_modulus_policy", C.c_char * 128),
        ("accumulator_safety_status", C.c_char * 128),
    ]


class GroupedGemmTask(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint64),
        ("abi_version", C.c_uint32),
        ("a", C.c_void_p),
        ("b", C.c_void_p),
        ("c", C.c_void_p),
        ("workspace", C.c_void_p),
    ]


class GroupedDispatchContractInfo(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint64),
        ("abi_version", C.c_uint32),
        ("backend", C.c_uint32),
        ("semantics", C.c_uint32),
        ("task_count", C.c_uint32),
    ] + [(name, C.c_uint32) for name in (
        "descriptor_contract_supported", "public_execution_available", "same_shape_required",
        "same_semantics_required", "compact_row_major_required", "unique_matrix_handles_required",
        "unique_workspace_handles_required", "same_plan_fingerprint_required", "same_device_required",
        "device_resident_inputs_required", "per_task_source_versions_required", "produces_device_current_output",
        "final_export_required_for_host_output", "per_task_status_required", "checksum_policy_required",
        "descriptor_reuse_validated", "flags")] + [
        ("descriptor_layout", C.c_char * 96),
        ("bucket_policy", C.c_char * 96),
        ("source_version_policy", C.c_char * 96),
        ("workspace_policy", C.c_char * 96),
        ("matrix_ownership_policy", C.c_char * 128),
        ("descriptor_reuse_policy", C.c_char * 128),
        ("stride_policy", C.c_char * 128),
        ("output_currentness_policy", C.c_char * 128),
        ("lifetime_policy", C.c_char * 128),
        ("checksum_policy", C.c_char * 96),
        ("status_policy", C.c_char * 96),
        ("device_descriptor_policy", C.c_char * 96),
        ("output_domain", C.c_char * 64),
        ("unsupported_reason", C.c_char * 160),
        ("detail", C.c_char * 256),
    ]


class BackendCapabilityInfo(C.Structure):
    """rns8_backend_capability_info (rns8.h)."""
    _fields_ = [
        ("struct_size", C.c_uint64),
        ("abi_version", C.c_uint32),
        ("backend", C.c_uint32),
    ] + [(name, C.c_uint32) for name in (
        "is_accelerator", "is_available", "is_correctness_backend", "is_matrix_engine_backend",
        "supports_bounded_rns", "supports_exact_wide_rns", "supports_finite_u8", "supports_wrap64",
        "requires_feature_detection", "enable_flag_fail_fast", "candidate_evidence_only",
        "compiled_kernel_available", "exact_differential_validated", "performance_validated", "flags")] + [
        ("backend_name", C.c_char * 64),
        ("selected_kernel", C.c_char * 128),
        ("library_name", C.c_char * 64),
        ("library_version", C.c_char * 64),
        ("enable_flag", C.c_char * 64),
        ("epilogue_mode", C.c_char * 96),
        ("workspace_mode", C.c_char * 96),
        ("isa_evidence", C.c_char * 128),
        ("status", C.c_char * 128),
        ("detail", C.c_char * 256),
    ]


class PlanPackingInfo(C.Structure):
    """rns8_plan_packing_info (rns8.h)."""
    _fields_ = [
        ("struct_size", C.c_uint64),
        ("abi_version", C.c_uint32),
        ("backend", C.c_uint32),
        ("semantics", C.c_uint32),
    ] + [(name, C.c_uint32) for name in (
        "uses_resident_matrix_inputs", "uses_transient_pack_workspace", "uses_matrix_engine_pack_layout",
        "reusable_prepack_cache_available", "production_prepack_cache_available", "flags", "input_domain",
        "output_domain", "output_host_current", "output_device_current", "next_op_flags", "reserved0")] + [
        (name, C.c_uint64) for name in (
            "a_pack_workspace_bytes", "b_pack_workspace_bytes", "accumulator_workspace_bytes",
            "library_workspace_bytes", "total_transient_workspace_bytes")] + [
        ("input_domain_name", C.c_char * 64),
        ("output_domain_name", C.c_char * 64),
        ("next_op_hint", C.c_char * 160),
        ("a_layout_version", C.c_char * 96),
        ("b_layout_version", C.c_char * 96),
        ("output_layout_version", C.c_char * 96),
        ("prepack_cache_scope", C.c_char * 96),
        ("detail", C.c_char * 256),
    ]


class ResidentLifetimeInfo(C.Structure):
    """rns8_resident_lifetime_info (rns8.h)."""
    _fields_ = [
        ("struct_size", C.c_uint64),
        ("abi_version", C.c_uint32),
    ] + [(name, C.c_uint32) for name in (
        "backend", "semantics", "logical_layout", "bound_kind", "matrix_role", "current_output_domain")] + [
        ("rows", C.c_int64),
        ("cols", C.c_int64),
        ("logical_ld", C.c_int64),
        ("max_prefix", C.c_uint32),
        ("finite_modulus", C.c_uint32),
        ("source_version", C.c_uint64),
        ("plan_fingerprint", C.c_uint64),
        ("workspace_fingerprint", C.c_uint64),
        ("hip_device_id", C.c_int32),
    ] + [(name, C.c_uint32) for name in (
        "source_version_valid", "host_current", "device_current", "device_resident", "plan_binding_available",
        "plan_binding_matches", "workspace_binding_available", "workspace_identity_matches",
        "workspace_schedule_matches", "workspace_backend_matches", "workspace_binding_matches",
        "device_id_matches", "can_feed_rns_gemm", "can_feed_native_gemm", "can_feed_final_export", "flags")] + [
        ("current_domain", C.c_char * 64),
        ("matrix_role_name", C.c_char * 32),
        ("source_version_policy", C.c_char * 96),
        ("workspace_binding_policy", C.c_char * 128),
        ("output_currentness_policy", C.c_char * 128),
        ("lifetime_policy", C.c_char * 128),
        ("mismatch_policy", C.c_char * 160),
        ("detail", C.c_char * 256),
    ]


def new_struct(cls):
    s = cls()
    s.struct_size = C.sizeof(cls)
    s.abi_version = ABI_VERSION
    return s


_P = C.c_void_p
_I64 = C.c_int64
_U64 = C.c_uint64
_U32 = C.c_uint32
_U16 = C.c_uint16

# name -> (restype, argtypes)
PROTOTYPES = {
    "rns8_status_string": (C.c_char_p, [_U32]),
    "rns8_default_modulus_count": (_U32, []),
    "rns8_default_modulus": (_U16, [_U32]),
    "rns8_prefix_range_bits": (C.c_double, [_U32]),
    "rns8_validate_default_moduli": (_U32, []),
    "rns8_create_context": (_U32, [C.c_int, C.POINTER(ContextOptions), C.POINTER(_P)]),
    "rns8_destroy_context": (_U32, [_P]),
    "rns8_get_device_info": (_U32, [_P, C.POINTER(DeviceInfo)]),
    "rns8_create_plan": (_U32, [_P, C.POINTER(GemmDesc), C.POINTER(_P)]),
    "rns8_destroy_plan": (_U32, [_P]),
    "rns8_get_plan_schedule_info": (_U32, [_P, C.POINTER(PlanScheduleInfo)]),
    "rns8_create_workspace": (_U32, [_P, _P, C.POINTER(_P)]),
    "rns8_destroy_workspace": (_U32, [_P]),
    "rns8_create_matrix": (_U32, [_P, C.POINTER(MatrixDesc), C.POINTER(_P)]),
    "rns8_destroy_matrix": (_U32, [_P]),
    "rns8_get_matrix_storage_info": (_U32, [_P, C.POINTER(MatrixStorageInfo)]),
    "rns8_pack_i64": (_U32, [_P, _P, _P, _I64, _U64]),
    "rns8_pack_u64": (_U32, [_P, _P, _P, _I64, _U64]),
    "rns8_pack_finite_u8": (_U32, [_P, _P, _U16, _P, _I64, _U64]),
    "rns8_gemm_rns": (_U32, [_P, _P, _P, _P, _P, _P]),
    "rns8_gemm_finite_u8": (_U32, [_P, _P, _U16, _P, _P, _P, _P]),
    "rns8_export_i64": (_U32, [_P, _P, _P, _P, _I64]),
    "rns8_export_u64": (_U32, [_P, _P, _P, _P, _I64]),
    "rns8_export_finite_u8": (_U32, [_P, _P, _U16, _P, _P, _I64]),
    "rns8_export_exact_wide_signed_limbs": (_U32, [_P, _P, _P, _P, _I64, _U32]),
    "rns8_export_exact_wide_unsigned_limbs": (_U32, [_P, _P, _P, _P, _I64, _U32]),
    "rns8_gemm_i64_oneshot": (_U32, [_P, C.POINTER(GemmDesc), _P, _I64, _P, _I64, _P, _I64]),
    "rns8_gemm_u64_oneshot": (_U32, [_P, C.POINTER(GemmDesc), _P, _I64, _P, _I64, _P, _I64]),
    "rns8_gemm_finite_ring_u8_oneshot": (_U32, [_P, C.POINTER(GemmDesc), _U16, _P, _I64, _P, _I64, _P, _I64]),
    "rns8_gemm_finite_field_u8_oneshot": (_U32, [_P, C.POINTER(GemmDesc), _U16, _P, _I64, _P, _I64, _P, _I64]),
    "rns8_mi355x_select_prefix": (_U32, [C.POINTER(GemmDesc), C.POINTER(_U32)]),
    "rns8_mi355x_plan_schedule": (_U32, [C.POINTER(GemmDesc), C.POINTER(PlanScheduleInfo), _P, _U64,
                                         C.POINTER(_U64)]),
    "rns8_get_plan_tile_schedule": (_U32, [_P, _P, _U64, C.POINTER(_U64)]),
    "rns8_mi355x_pack_i64_device": (_U32, [_P, _P, _P, _I64, _U64, _P]),
    "rns8_mi355x_pack_u64_device": (_U32, [_P, _P, _P, _I64, _U64, _P]),
    "rns8_mi355x_pack_finite_u8_device": (_U32, [_P, _P, _U16, _P, _I64, _U64, _P]),
    "rns8_mi355x_gemm_rns_async": (_U32, [_P, _P, _P, _P, _P, _P, _P]),
    "rns8_mi355x_gemm_rns_noalloc": (_U32, [_P, _P, _P, _P, _P, _P]),
    "rns8_mi355x_gemm_native_i64_async": (_U32, [_P, _P, _P, _I64, _P, _I64, _P, _P, _P]),
    "rns8_mi355x_gemm_native_u64_async": (_U32, [_P, _P, _P, _I64, _P, _I64, _P, _P, _P]),
    "rns8_mi355x_gemm_finite_u8_async": (_U32, [_P, _P, _U16, _P, _P, _P, _P, _P]),
    "rns8_mi355x_export_i64_device": (_U32, [_P, _P, _P, _P, _I64, _P, _P]),
    "rns8_mi355x_export_u64_device": (_U32, [_P, _P, _P, _P, _I64, _P, _P]),
    "rns8_mi355x_export_exact_wide_signed_limbs_device": (_U32, [_P, _P, _P, _P, _I64, _U32, _P, _P]),
    "rns8_mi355x_export_exact_wide_unsigned_limbs_device": (_U32, [_P, _P, _P, _P, _I64, _U32, _P, _P]),
    "rns8_mi355x_export_finite_u8_device": (_U32, [_P, _P, _U16, _P, _P, _I64, _P]),
    "rns8_get_plan_backend_info": (_U32, [_P, C.POINTER(PlanBackendInfo)]),
    "rns8_gemm_rns_grouped": (_U32, [_P, _P, C.POINTER(GroupedGemmTask), _U32]),
    "rns8_gemm_finite_u8_grouped": (_U32, [_P, _P, _U16, C.POINTER(GroupedGemmTask), _U32]),
    "rns8_mi355x_gemm_rns_grouped_async": (_U32, [_P, _P, C.POINTER(GroupedGemmTask), _U32, _P]),
    "rns8_mi355x_gemm_finite_u8_grouped_async": (_U32, [_P, _P, _U16, C.POINTER(GroupedGemmTask), _U32, _P]),
    "rns8_get_grouped_dispatch_contract_info": (_U32, [_P, _U32, C.POINTER(GroupedDispatchContractInfo)]),
    "rns8_get_backend_capability_info": (_U32, [_U32, C.POINTER(BackendCapabilityInfo)]),
    "rns8_get_plan_packing_info": (_U32, [_P, C.POINTER(PlanPackingInfo)]),
    "rns8_get_resident_lifetime_info": (_U32, [_P, _P, _P, _U32, C.POINTER(ResidentLifetimeInfo)]),
    "rns8_mi355x_get_matrix_planes": (_U32, [_P, C.POINTER(_P), C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_U32)]),
    "rns8_mi355x_get_exact_proof": (_U32, [_P, _P, _P, C.POINTER(_U32), _P, _P]),
}

LIB_PATH = Path(__file__).resolve().parent / "librns8.so"


def load_library(path: Path | None = None) -> C.CDLL:
    """Load librns8.so and bind prototypes. Raises if the library is missing:
    there is no fallback implementation."""
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(f"{p} is missing: build it with rns8_amd/build.py (hipcc, gfx950)")
    lib = C.CDLL(str(p))
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib
