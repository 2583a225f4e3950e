/* MI355X extensions to the rns8 C ABI: the device-resident hot path.
 *
 * The reference ABI (rns8/rns8.h) takes and returns host memory and ends
 * every call with a device synchronization, so each GEMM pays PCIe transfers.
 * These entry points run the same pack -> plane GEMM -> Garner stages on
 * operands that already live in HBM, enqueue their kernels on a caller
 * stream and return without synchronizing. They have no counterpart in the
 * reference; they are what a caller that chains GEMMs on the GPU (or a
 * benchmark measuring the kernels rather than PCIe) binds. They reuse the
 * same handles, validation and kernels as the host entry points.
 *
 * Conventions
 *   - `stream` is a hipStream_t passed as void*; NULL selects the context's
 *     own stream. Work is ordered on that stream only.
 *   - Device pointers must be accessible from the context's device.
 *   - Range violations are reported through `d_status`: a device uint32_t
 *     that the caller zeroes before the call; the export kernel sets it
 *     nonzero if any cell violates the contract. The output contents of such
 *     a call are unspecified (the host exports keep `dst` untouched instead).
 *   - Validation failures return before anything is enqueued.
 */
#ifndef RNS8_MI355X_H
#define RNS8_MI355X_H

#include <stdint.h>

#include "rns8/rns8.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Prefix a plan created from `desc` would select (validation and prefix
 * selection of rns8_create_plan, reference api_plan_public_api.inc:3-73 and
 * api_plan_schedule.inc:263-278), without a context or device. Finite
 * semantics report 0. */
RNS8_API rns8_status rns8_mi355x_select_prefix(const rns8_gemm_desc* desc, uint32_t* out_prefix);

/* The schedule rns8_create_plan would build for `desc`, without a context or
 * device: the same results as rns8_get_plan_schedule_info and
 * rns8_get_plan_tile_schedule on that plan (reference rns8.h:683-691,
 * api_plan_schedule.inc:109-279, api_plan_public_api.inc:80-160), including
 * per-tile bounded schedules. `entries` may be NULL to query the count. */
RNS8_API rns8_status rns8_mi355x_plan_schedule(
    const rns8_gemm_desc* desc,
    rns8_plan_schedule_info* info,
    rns8_plan_tile_schedule_entry* entries,
    uint64_t capacity,
    uint64_t* written);

/* Device-source variants of rns8_pack_i64 / rns8_pack_u64 / rns8_pack_finite_u8
 * (reference rns8.h:848-911): `d_src` is device memory, row stride `ld`
 * elements. For exact-wide matrices the magnitude proof is the one the
 * reference's host pack builds (per-row and per-column maxima, sums,
 * absolute sums, extremes and deviation sums, reference exact_range.hpp
 * :52-78), computed on the GPU; so every later admission equals the one
 * the reference makes for the same values. At prefix 9 and up the call does
 * not synchronize; below, it reads max |x| back before writing anything. */
RNS8_API rns8_status rns8_mi355x_pack_i64_device(
    rns8_context* ctx,
    rns8_matrix* matrix,
    const int64_t* d_src,
    int64_t ld,
    uint64_t source_version,
    void* stream);
RNS8_API rns8_status rns8_mi355x_pack_u64_device(
    rns8_context* ctx,
    rns8_matrix* matrix,
    const uint64_t* d_src,
    int64_t ld,
    uint64_t source_version,
    void* stream);
RNS8_API rns8_status rns8_mi355x_pack_finite_u8_device(
    rns8_context* ctx,
    rns8_matrix* matrix,
    uint16_t modulus,
    const uint8_t* d_src,
    int64_t ld,
    uint64_t source_version,
    void* stream);

/* Asynchronous rns8_gemm_rns / rns8_gemm_finite_u8 (reference rns8.h:988,
 * 1098): same validation and admission, kernels enqueued on `stream`.
 * Exact-wide admission: the call decides on k * maxA * maxB, from maxima the
 * host already holds, and does not synchronize when that bound fits. When it
 * does not fit, the reference's refined bound (the minimum of its candidate
 * bounds for every output cell, from the operands' per-row and per-column
 * summaries) is computed on the device and read back before the call
 * returns: the call then synchronizes `stream`. */
RNS8_API rns8_status rns8_mi355x_gemm_rns_async(
    rns8_context* ctx,
    const rns8_plan* plan,
    const rns8_matrix* A,
    const rns8_matrix* B,
    rns8_matrix* C,
    rns8_workspace* workspace,
    void* stream);
RNS8_API rns8_status rns8_mi355x_gemm_finite_u8_async(
    rns8_context* ctx,
    const rns8_plan* plan,
    uint16_t modulus,
    const rns8_matrix* A,
    const rns8_matrix* B,
    rns8_matrix* C,
    rns8_workspace* workspace,
    void* stream);

/* rns8_mi355x_gemm_rns_async for bounded int64 / uint64 plans (global or
 * per-tile bounds) without a workspace, for callers that cannot allocate:
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation. No counterpart in the reference. The call allocates nothing,
 * on the device or the host: split-K residues (shapes with few output tiles
 * and a long K) go to a static per-device scratch array of 4 MiB that the
 * library holds until the process ends (its address is looked up when a
 * context is created). Plans whose split-K residues exceed 4 MiB return
 * RNS8_WORKSPACE_TOO_SMALL;
 * exact-wide plans return RNS8_UNSUPPORTED_BACKEND (their admission may read
 * a device bound back and keeps its proofs in host memory). Every call on one device shares that device's
 * scratch: calls that overlap on one device (on different streams, or from
 * several threads) race and must be ordered by the caller; calls ordered on
 * one stream do not. Results equal rns8_mi355x_gemm_rns_async's. */
RNS8_API rns8_status rns8_mi355x_gemm_rns_noalloc(
    rns8_context* ctx,
    const rns8_plan* plan,
    const rns8_matrix* A,
    const rns8_matrix* B,
    rns8_matrix* C,
    void* stream);

/* Stream-ordered rns8_gemm_rns_grouped / rns8_gemm_finite_u8_grouped
 * (reference rns8.h:1061-1065, 1139-1144): the same validation, the group
 * enqueued on `stream` as one persistent launch per 65536-K block and up to
 * 32 tasks. */
RNS8_API rns8_status rns8_mi355x_gemm_rns_grouped_async(
    rns8_context* ctx,
    const rns8_plan* plan,
    const rns8_grouped_gemm_task* tasks,
    uint32_t task_count,
    void* stream);
RNS8_API rns8_status rns8_mi355x_gemm_finite_u8_grouped_async(
    rns8_context* ctx,
    const rns8_plan* plan,
    uint16_t modulus,
    const rns8_grouped_gemm_task* tasks,
    uint32_t task_count,
    void* stream);

/* Fused native-input GEMM for bounded int64 / uint64 plans: C's residue
 * planes straight from native device operands (m x k at row stride lda, k x n
 * at row stride ldb, in elements), the pack folded into the GEMM's operand
 * loads, enqueued on `stream` (reference hip_direct_gemm_native_kernels.cuh:
 * 9-193, its native-operand GEMM behind the oneshot path,
 * hip_backend_gemm_native_prefix.inc). Offered for outputs small enough that
 * the product is split along K, with 16-byte aligned operands and even row
 * strides below 2^21 elements; returns RNS8_UNSUPPORTED_BACKEND otherwise
 * (such plans pack their operands once and multiply with rns8_gemm_rns). The
 * plan's declared bound covers the result exactly as for rns8_gemm_rns. */
RNS8_API rns8_status rns8_mi355x_gemm_native_i64_async(
    rns8_context* ctx,
    const rns8_plan* plan,
    const int64_t* d_A,
    int64_t lda,
    const int64_t* d_B,
    int64_t ldb,
    rns8_matrix* C,
    rns8_workspace* workspace,
    void* stream);
RNS8_API rns8_status rns8_mi355x_gemm_native_u64_async(
    rns8_context* ctx,
    const rns8_plan* plan,
    const uint64_t* d_A,
    int64_t lda,
    const uint64_t* d_B,
    int64_t ldb,
    rns8_matrix* C,
    rns8_workspace* workspace,
    void* stream);

/* Device-destination variants of the exports (reference rns8.h:1146-1242). */
RNS8_API rns8_status rns8_mi355x_export_i64_device(
    rns8_context* ctx,
    const rns8_plan* plan,
    const rns8_matrix* C,
    int64_t* d_dst,
    int64_t ld,
    uint32_t* d_status,
    void* stream);
RNS8_API rns8_status rns8_mi355x_export_u64_device(
    rns8_context* ctx,
    const rns8_plan* plan,
    const rns8_matrix* C,
    uint64_t* d_dst,
    int64_t ld,
    uint32_t* d_status,
    void* stream);
RNS8_API rns8_status rns8_mi355x_export_exact_wide_signed_limbs_device(
    rns8_context* ctx,
    const rns8_plan* plan,
    const rns8_matrix* C,
    uint64_t* d_dst,
    int64_t ld,
    uint32_t limb_count,
    uint32_t* d_status,
    void* stream);
RNS8_API rns8_status rns8_mi355x_export_exact_wide_unsigned_limbs_device(
    rns8_context* ctx,
    const rns8_plan* plan,
    const rns8_matrix* C,
    uint64_t* d_dst,
    int64_t ld,
    uint32_t limb_count,
    uint32_t* d_status,
    void* stream);
RNS8_API rns8_status rns8_mi355x_export_finite_u8_device(
    rns8_context* ctx,
    const rns8_plan* plan,
    uint16_t modulus,
    const rns8_matrix* C,
    uint8_t* d_dst,
    int64_t ld,
    void* stream);

/* Layout of a resident matrix's planes in HBM ("rns8_mi355x_planes_v1"):
 * plane p, row r, column c lives at d_planes + p*plane_pitch + r*row_pitch + c
 * as a centered int8 residue; padding bytes are zero. Lets device code read
 * or produce residue planes directly. */
RNS8_API rns8_status rns8_mi355x_get_matrix_planes(
    const rns8_matrix* matrix,
    void** d_planes,
    int64_t* row_pitch,
    int64_t* plane_pitch,
    uint32_t* plane_count);

/* One row or column of an exact-wide matrix's magnitude proof, as
 * little-endian 64-bit words (reference rns8_exact_axis_range,
 * internal.hpp:72-86). */
typedef struct rns8_mi355x_exact_axis {
  uint64_t max_magnitude[4]; /* unsigned 256-bit */
  uint64_t absolute_sum[4];  /* unsigned 256-bit */
  uint64_t sum[2];           /* signed 128-bit, two's complement */
  uint64_t minimum[2];       /* signed 128-bit */
  uint64_t maximum[2];       /* signed 128-bit */
  uint64_t deviation_sum[2]; /* unsigned 128-bit */
} rns8_mi355x_exact_axis;

#define RNS8_MI355X_EXACT_AXES_NATIVE 0u  /* a pack's summaries: every field */
#define RNS8_MI355X_EXACT_AXES_CARRIED 1u /* a GEMM result's: max_magnitude, absolute_sum */
#define RNS8_MI355X_EXACT_AXES_NONE 2u    /* no per-axis summaries */

/* The magnitude proof an exact-wide matrix carries into later GEMMs
 * (reference exact_range.hpp:51-171): its bound (max |x| of a packed
 * operand, the proven bound of a GEMM result) into bound[0..3] as an
 * unsigned 256-bit integer, the kind of its axes, and rows[desc.rows] /
 * cols[desc.cols] (either may be NULL; untouched for
 * RNS8_MI355X_EXACT_AXES_NONE). A result's own summaries are computed when
 * first needed, here on the context's stream. Synchronizes. No counterpart
 * in the reference's C API (its proof is internal state). Returns
 * RNS8_INVALID_ARGUMENT for matrices without an exact-wide proof. */
RNS8_API rns8_status rns8_mi355x_get_exact_proof(
    rns8_context* ctx,
    const rns8_matrix* matrix,
    uint64_t bound[4],
    uint32_t* axes_kind,
    rns8_mi355x_exact_axis* rows,
    rns8_mi355x_exact_axis* cols);

#ifdef __cplusplus
}
#endif

#endif /* RNS8_MI355X_H */
