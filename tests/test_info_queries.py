"""The reference's informational queries through the C ABI:
rns8_get_backend_capability_info (reference src/core/api_backend_info.cpp:407),
rns8_get_plan_packing_info (src/core/api_plan_public_api.inc:370) and
rns8_get_resident_lifetime_info (src/core/api_resident_lifetime_public_api.inc:137).

The record layouts are the reference header's (the ctypes records in
rns8_amd/abi.py carry the same sizes, and a wrong struct_size is refused).
Checked: the argument validation the reference applies (null records, bad
struct_size, out-of-range backend or role, a workspace without a plan), the
fields that follow from this library (HIP_DIRECT and AUTO are the executing
backends, every other backend reports itself unsupported), the currentness of
matrices no pack or GEMM has written yet, and the bindings a
resident matrix reports against plans and workspaces: the role's shape must
match the plan, a workspace must belong to the plan, and a matrix becomes
device-current, with its source version, once packed.
"""
import ctypes as C

import numpy as np
import pytest

import rns8_amd as r
from rns8_amd import abi, inputs

OURS = (abi.BACKEND_AUTO, abi.BACKEND_HIP_DIRECT)
LAST_BACKEND = 8  # RNS8_BACKEND_AMDGPU_BUILTINS


def _capability(backend, size=None):
    info = abi.new_struct(abi.BackendCapabilityInfo)
    if size is not None:
        info.struct_size = size
    return r.lib().rns8_get_backend_capability_info(backend, C.byref(info)), info


@pytest.mark.parametrize("backend", range(LAST_BACKEND + 1))
def test_backend_capability(backend):
    st, info = _capability(backend)
    assert st == r.SUCCESS
    assert info.backend == backend
    ours = backend in OURS
    for field in ("is_accelerator", "is_matrix_engine_backend", "supports_bounded_rns", "supports_exact_wide_rns",
                  "supports_finite_u8", "compiled_kernel_available"):
        assert getattr(info, field) == (1 if ours else 0), field
    assert info.supports_wrap64 == 0  # wrap64 is outside this library
    assert info.library_name == b"rns8_mi355x"
    if ours:
        assert info.is_available == (1 if info.status == b"available" else 0)
        assert info.status in (b"available", b"no_hip_device")
    else:
        assert info.is_available == 0 and info.status == b"unsupported_backend"


def test_backend_capability_validation():
    assert _capability(LAST_BACKEND + 1)[0] == r.INVALID_ARGUMENT
    assert _capability(abi.BACKEND_HIP_DIRECT, size=C.sizeof(abi.BackendCapabilityInfo) - 8)[0] == \
        r.INVALID_ARGUMENT
    assert r.lib().rns8_get_backend_capability_info(abi.BACKEND_HIP_DIRECT, None) == r.INVALID_ARGUMENT


@pytest.mark.gpu
def test_backend_capability_available_on_gpu(gpu_ctx):
    st, info = _capability(abi.BACKEND_HIP_DIRECT)
    assert st == r.SUCCESS and info.is_available == 1 and info.status == b"available"


def _packing(plan, size=None):
    info = abi.new_struct(abi.PlanPackingInfo)
    if size is not None:
        info.struct_size = size
    return r.lib().rns8_get_plan_packing_info(plan.ptr if plan else None, C.byref(info)), info


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k", [(256, 256, 256), (128, 128, 65536)])
def test_plan_packing_bounded(gpu_ctx, m, n, k):
    plan = r.Plan(gpu_ctx, r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, m, n, k, bound=1 << 60))
    st, info = _packing(plan)
    assert st == r.SUCCESS
    assert info.semantics == r.BOUNDED_I64 and info.backend == abi.BACKEND_HIP_DIRECT
    assert info.uses_resident_matrix_inputs == 1 and info.output_device_current == 1
    assert info.input_domain == info.output_domain == 1  # RNS8_OUTPUT_DOMAIN_RNS_RESIDUE
    assert info.next_op_flags == 0b11  # final export, or another rns8_gemm_rns
    # the split-K residue slots are the only transient workspace
    assert info.accumulator_workspace_bytes == plan.backend_info().workspace_required_bytes
    assert info.total_transient_workspace_bytes == info.accumulator_workspace_bytes
    if k > 65536 // 2:
        assert info.accumulator_workspace_bytes > 0
    assert info.a_layout_version == info.b_layout_version == info.output_layout_version == b"rns8_mi355x_planes_v1"


@pytest.mark.gpu
def test_plan_packing_finite_and_validation(gpu_ctx):
    plan = r.Plan(gpu_ctx, r.gemm_desc(r.FINITE_FIELD_U8, r.BOUND_NONE, 64, 64, 64, finite_modulus=251))
    st, info = _packing(plan)
    assert st == r.SUCCESS and info.semantics == r.FINITE_FIELD_U8
    assert info.input_domain == info.output_domain == 3  # RNS8_OUTPUT_DOMAIN_FINITE_U8
    assert _packing(None)[0] == r.INVALID_ARGUMENT
    # records at least the expected size are accepted (later ABI revisions
    # append fields), shorter ones refused
    assert _packing(plan, size=C.sizeof(abi.PlanPackingInfo) - 8)[0] == r.INVALID_ARGUMENT
    assert _packing(plan, size=C.sizeof(abi.PlanPackingInfo) + 8)[0] == r.SUCCESS


def _lifetime(matrix, plan, ws, role):
    info = abi.new_struct(abi.ResidentLifetimeInfo)
    st = r.lib().rns8_get_resident_lifetime_info(matrix.ptr if matrix else None, plan.ptr if plan else None,
                                                 ws.ptr if ws else None, role, C.byref(info))
    return st, info


@pytest.mark.gpu
def test_resident_lifetime_bindings(gpu_ctx):
    m, n, k = 48, 80, 64
    sem, bk = r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS
    plan = r.Plan(gpu_ctx, r.gemm_desc(sem, bk, m, n, k, bound=1 << 50))
    other = r.Plan(gpu_ctx, r.gemm_desc(sem, bk, m, n, k + 1, bound=1 << 50))
    p = plan.prefix
    mk = lambda rows, cols: r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, sem, bk, p))
    A, B, Cm = mk(m, k), mk(k, n), mk(m, n)
    ws, ws_other = r.Workspace(gpu_ctx, plan), r.Workspace(gpu_ctx, other)

    st, info = _lifetime(A, plan, ws, 1)
    assert st == r.SUCCESS
    assert (info.rows, info.cols, info.matrix_role, info.semantics) == (m, k, 1, sem)
    assert info.matrix_role_name == b"a"
    assert info.plan_binding_available == info.plan_binding_matches == 1
    assert info.workspace_binding_available == info.workspace_identity_matches == 1
    assert info.workspace_binding_matches == 1
    # not packed yet: nothing current on the device, no source version
    assert info.device_current == 0 and info.source_version_valid == 0 and info.can_feed_rns_gemm == 0
    assert info.device_resident == 1

    # each operand matches the plan in its own role only (48 x 64 is neither B nor C here)
    for matrix, role, want in ((A, 1, 1), (A, 2, 0), (A, 3, 0), (B, 2, 1), (B, 1, 0), (Cm, 3, 1), (Cm, 2, 0)):
        st, info = _lifetime(matrix, plan, None, role)
        assert st == r.SUCCESS and info.plan_binding_matches == want, (role, want)
        assert info.workspace_binding_available == 0

    # a workspace of another plan does not bind
    st, info = _lifetime(A, plan, ws_other, 1)
    assert st == r.SUCCESS and info.workspace_identity_matches == 0 and info.workspace_binding_matches == 0

    # packed with a source version: device-current, version reported
    src = inputs.int_range(3, (m, k), 20)
    r.check(r.pack_i64(gpu_ctx, A, src, 5), "pack")
    st, info = _lifetime(A, None, None, 1)
    assert st == r.SUCCESS and info.plan_binding_available == 0
    assert info.device_current == 1 and info.can_feed_rns_gemm == 1 and info.can_feed_final_export == 1
    assert info.source_version == 5 and info.source_version_valid == 1
    assert info.current_domain == b"rns_residue"

    # validation: no matrix, a workspace without a plan, a role past C, a bad record size
    assert _lifetime(None, plan, None, 1)[0] == r.INVALID_ARGUMENT
    assert _lifetime(A, None, ws, 1)[0] == r.INVALID_ARGUMENT
    assert _lifetime(A, plan, None, 4)[0] == r.INVALID_ARGUMENT
    bad = abi.new_struct(abi.ResidentLifetimeInfo)
    bad.struct_size = 16
    assert r.lib().rns8_get_resident_lifetime_info(A.ptr, None, None, 1, C.byref(bad)) == r.INVALID_ARGUMENT
    np.testing.assert_array_equal(A.read_residues()[0], np.asarray(src % 256, dtype=np.int64).astype(np.int8))


@pytest.mark.gpu
@pytest.mark.parametrize("finite", [False, True])
def test_unwritten_matrices_are_not_current(gpu_ctx, finite):
    """A matrix holds no current residues until a pack or a GEMM writes them
    (reference internal.hpp:106, api_matrix_currentness_storage.inc:339): a
    GEMM with a never-packed operand and an export of a never-computed
    result are refused with RNS8_INVALID_ARGUMENT (api_gemm.cpp:101-104,
    api_export.cpp:39 and :78), and both work once the planes are written."""
    m, n, k = 20, 24, 16
    if finite:
        sem, bk, p, mod = r.FINITE_RING_U8, r.BOUND_NONE, 0, 97
        plan = r.Plan(gpu_ctx, r.gemm_desc(sem, bk, m, n, k, finite_modulus=mod))
    else:
        sem, bk, mod = r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, 0
        plan = r.Plan(gpu_ctx, r.gemm_desc(sem, bk, m, n, k, bound=1 << 40))
        p = plan.prefix
    mk = lambda rows, cols: r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, sem, bk, p))
    A, B, Cm = mk(m, k), mk(k, n), mk(m, n)
    ws = r.Workspace(gpu_ctx, plan)
    gemm = (lambda: r.gemm_finite_u8(gpu_ctx, plan, mod, A, B, Cm, ws)) if finite else \
        (lambda: r.gemm_rns(gpu_ctx, plan, A, B, Cm, ws))
    out = np.full((m, n), 7, dtype=np.uint8 if finite else np.int64)
    export = (lambda: r.export_finite_u8(gpu_ctx, plan, mod, Cm, out)) if finite else \
        (lambda: r.export_i64(gpu_ctx, plan, Cm, out))
    assert _lifetime(A, None, None, 1)[1].device_current == 0
    assert export() == r.INVALID_ARGUMENT and (out == 7).all()
    if finite:
        a = inputs.bytes_below(5, (m, k), 256)
        b = inputs.bytes_below(6, (k, n), 256)
        r.check(r.pack_finite_u8(gpu_ctx, A, mod, a, 1), "pack A")
        assert gemm() == r.INVALID_ARGUMENT  # B never packed
        r.check(r.pack_finite_u8(gpu_ctx, B, mod, b, 2), "pack B")
        want = ((a.astype(np.int64) @ b.astype(np.int64)) % mod).astype(np.uint8)
    else:
        a = inputs.int_range(5, (m, k), 18)
        b = inputs.int_range(6, (k, n), 18)
        r.check(r.pack_i64(gpu_ctx, A, a, 1), "pack A")
        assert gemm() == r.INVALID_ARGUMENT  # B never packed
        r.check(r.pack_i64(gpu_ctx, B, b, 2), "pack B")
        want = a @ b
    assert export() == r.INVALID_ARGUMENT  # C not computed yet
    r.check(gemm(), "gemm")
    r.check(export(), "export")
    np.testing.assert_array_equal(out, want)
