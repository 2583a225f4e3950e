// rns8 ABI execution: pack, plane GEMM, export and one-shot entry points,
// plus the device-resident MI355X extensions (rns8_mi355x.h).
//
// Order of checks and statuses follows the reference:
//   rns8_pack_*            src/core/api_pack.cpp:31-305
//   rns8_gemm_rns          src/core/api_gemm.cpp:50-111, 838-983
//   rns8_gemm_finite_u8    src/core/api_gemm.cpp:113-160, 1281-1330
//   rns8_export_*          src/core/api_export.cpp:5-53, 307-803
//   one-shot               src/core/api_oneshot.cpp:78-133, 440-677
//   exact-wide proofs      src/core/exact_range.hpp:16-171
// Kernels run on the context's stream (or the caller's, for the extensions);
// host entry points synchronize before returning, like the reference.
#include <algorithm>
#include <cstring>
#include <exception>
#include <limits>
#include <thread>
#include <vector>

#include "contract.hpp"
#include "exact_proof.hpp"
#include "handles.hpp"
#include "kernels.hpp"

namespace rns8x {
namespace {

uint64_t output_source_version(uint64_t a, uint64_t b) {
  // reference api_plan_workspace_fingerprint.inc:18-23
  uint64_t h = 1469598103934665603ull;
  h ^= a;
  h *= 1099511628211ull;
  h ^= b;
  h *= 1099511628211ull;
  return h == 0 ? 1 : h;
}

// The largest magnitude a 64-bit operand can have: what a device-pointer
// pack's proof holds until it is read back.
I512 native_worst_case(rns8_semantics s) {
  return s == RNS8_EXACT_WIDE_SIGNED ? I512::pow2(63) : I512::from_u64(~uint64_t{0});
}

// ---- shared validation --------------------------------------------------------

rns8_status sync(hipStream_t s) { return hipStreamSynchronize(s) == hipSuccess ? RNS8_SUCCESS : RNS8_BACKEND_FAILURE; }

// ---- pack ------------------------------------------------------------------------

enum class Source { Host, Device };

template <typename T>
rns8_status pack_native(rns8_context* ctx, rns8_matrix* matrix, const T* src, int64_t ld, uint64_t sv, Source where,
                        void* stream_arg) {
  constexpr bool is_signed = std::is_same<T, int64_t>::value;
  if (!ctx || !matrix || !src) return RNS8_INVALID_ARGUMENT;
  const rns8_status chk = check_pack_native(*ctx, *matrix, ld, is_signed);
  if (chk != RNS8_SUCCESS) return chk;
  const rns8_semantics wide = is_signed ? RNS8_EXACT_WIDE_SIGNED : RNS8_EXACT_WIDE_UNSIGNED;
  const int64_t rows = matrix->desc.rows, cols = matrix->desc.cols;
  const bool same_source = sv != 0 && matrix->source_version == sv && matrix->device_current;
  const hipStream_t stream = pick_stream(*ctx, stream_arg);
  if (hipSetDevice(ctx->device_id) != hipSuccess) return RNS8_BACKEND_FAILURE;

  // exact-wide proof (api_pack.cpp:47-65), kept when the source is
  // unchanged: the operand's per-row and per-column summaries, computed on
  // the device into the matrix's free proof set and made current with the
  // planes. At prefix 9 and up (P > 2^64) every 64-bit operand is admitted,
  // so nothing waits for the proof and the host keeps a worst case of max |x|
  // (exact after a host-array pack, which synchronizes anyway). Smaller
  // prefixes need the maximum before anything is written (a refused pack
  // leaves the matrix as it was), so it is read back first.
  const bool is_wide = matrix->desc.semantics == wide;
  if (same_source) return RNS8_SUCCESS;
  const void* dsrc = src;
  int64_t dld = ld;
  if (where == Source::Host) {
    const std::size_t bytes = static_cast<std::size_t>(rows) * cols * sizeof(T);
    rns8_status st = ensure_device_buffer(ctx->device_id, &matrix->upload, &matrix->upload_bytes, bytes);
    if (st != RNS8_SUCCESS) return st;
    if (ctx->host.to_device(matrix->upload, src, cols * sizeof(T), ld * sizeof(T), rows, stream) != hipSuccess)
      return RNS8_BACKEND_FAILURE;
    dsrc = matrix->upload;
    dld = cols;
  }
  I512 proof_max;
  bool pending = false;
  if (is_wide) {
    rns8_status st = prove_native(*matrix, dsrc, dld, is_signed, stream);
    if (st != RNS8_SUCCESS) return st;
    const I512 worst = native_worst_case(matrix->desc.semantics);
    if (exact_range_fits(matrix->desc.semantics, worst, modulus_product(matrix->prefix))) {
      proof_max = worst;
      pending = true;
    } else {
      st = read_free_bound(*matrix, stream, proof_max);
      if (st != RNS8_SUCCESS) return st;
      if (!exact_range_fits(matrix->desc.semantics, proof_max, modulus_product(matrix->prefix)))
        return RNS8_RANGE_ERROR;
    }
  }
  const PackArgs args = pack_args(*matrix, dsrc, dld, is_signed);
  if (launch_pack_native(args, make_ladder_plane_consts(matrix->prefix), stream) != hipSuccess)
    return RNS8_BACKEND_FAILURE;
  if (is_wide) {
    const rns8_status st = commit_native_proof(*matrix, proof_max, pending, stream);
    if (st != RNS8_SUCCESS) return st;
  }
  if (where == Source::Host) {
    rns8_status st = sync(stream);
    if (st == RNS8_SUCCESS && is_wide && pending) st = resolve_exact_proof(*matrix, stream);
    if (st != RNS8_SUCCESS) return st;
  }
  matrix->device_current = true;
  matrix->source_version = sv;
  return RNS8_SUCCESS;
}

rns8_status pack_u8(rns8_context* ctx, rns8_matrix* matrix, uint16_t modulus, const uint8_t* src, int64_t ld,
                    uint64_t sv, Source where, void* stream_arg) {
  if (!ctx || !matrix || !src) return RNS8_INVALID_ARGUMENT;
  const rns8_status chk = check_pack_u8(*ctx, *matrix, modulus, ld);
  if (chk != RNS8_SUCCESS) return chk;
  if (sv != 0 && matrix->source_version == sv && matrix->finite_modulus == modulus && matrix->device_current)
    return RNS8_SUCCESS;
  const int64_t rows = matrix->desc.rows, cols = matrix->desc.cols;
  const hipStream_t stream = pick_stream(*ctx, stream_arg);
  if (hipSetDevice(ctx->device_id) != hipSuccess) return RNS8_BACKEND_FAILURE;
  const uint8_t* dsrc = src;
  int64_t dld = ld;
  if (where == Source::Host) {
    const std::size_t bytes = static_cast<std::size_t>(rows) * cols;
    rns8_status st = ensure_device_buffer(ctx->device_id, &matrix->upload, &matrix->upload_bytes, bytes);
    if (st != RNS8_SUCCESS) return st;
    if (ctx->host.to_device(matrix->upload, src, cols, ld, rows, stream) != hipSuccess) return RNS8_BACKEND_FAILURE;
    dsrc = static_cast<const uint8_t*>(matrix->upload);
    dld = cols;
  }
  const PackU8Args args = pack_u8_args(*matrix, dsrc, dld, modulus);
  if (launch_pack_u8(args, stream) != hipSuccess) return RNS8_BACKEND_FAILURE;
  if (where == Source::Host) {
    const rns8_status st = sync(stream);
    if (st != RNS8_SUCCESS) return st;
  }
  matrix->device_current = true;
  matrix->source_version = sv;
  matrix->finite_modulus = modulus;
  return RNS8_SUCCESS;
}

// ---- GEMM --------------------------------------------------------------------------

rns8_status run_gemm(rns8_context& ctx, const rns8_plan& plan, const rns8_matrix& A, const rns8_matrix& B,
                     rns8_matrix& C, int8_t* splitk_ws, uint32_t nplanes, const PlaneConsts& consts,
                     hipStream_t stream) {
  const GemmArgs g = gemm_args(plan, A, B, C, splitk_ws, nplanes, plan.splitk_slices);
  if (hipSetDevice(ctx.device_id) != hipSuccess) return RNS8_BACKEND_FAILURE;
  const hipError_t e = launch_gemm(g, consts, stream);
  if (e == hipErrorInvalidValue) return RNS8_UNSUPPORTED_BACKEND;  // shape outside the kernel's limits
  return e == hipSuccess ? RNS8_SUCCESS : RNS8_BACKEND_FAILURE;
}

// Per-tile plan whose schedule did not collapse: the listed GEMM over the
// plan's unit list plus the zero-output fills (the two write disjoint cells).
rns8_status run_gemm_tiled(rns8_context& ctx, const rns8_plan& plan, const rns8_matrix& A, const rns8_matrix& B,
                           rns8_matrix& C, hipStream_t stream) {
  const uint32_t planes = storage_prefix(plan);
  const GemmArgs g = gemm_args(plan, A, B, C, nullptr, planes, 1);
  if (hipSetDevice(ctx.device_id) != hipSuccess) return RNS8_BACKEND_FAILURE;
  hipError_t e = launch_gemm_listed(g, make_ladder_plane_consts(planes), plan.units, plan.unit_count,
                                    plan.unit_edge, stream);
  if (e == hipErrorInvalidValue) return RNS8_UNSUPPORTED_BACKEND;
  if (e == hipSuccess) e = launch_zero_tiles(C.planes, C.plane_ld, C.plane_pitch, plan.zero_fills,
                                             plan.zero_fill_count, stream);
  return e == hipSuccess ? RNS8_SUCCESS : RNS8_BACKEND_FAILURE;
}

rns8_status gemm_rns(rns8_context* ctx, const rns8_plan* plan, const rns8_matrix* A, const rns8_matrix* B,
                     rns8_matrix* C, rns8_workspace* ws, void* stream_arg, bool synchronous) {
  if (!ctx || !plan || !A || !B || !C || !ws) return RNS8_INVALID_ARGUMENT;
  rns8_status st = check_plan_ctx_ws(*ctx, *plan, *ws);
  if (st != RNS8_SUCCESS) return st;
  st = check_rns_operands(*ctx, *plan, *A, *B, *C);
  if (st != RNS8_SUCCESS) return st;
  const hipStream_t stream = pick_stream(*ctx, stream_arg);
  ExactAdmission adm;
  if (exact_wide(plan->desc.semantics)) {
    if (hipSetDevice(ctx->device_id) != hipSuccess) return RNS8_BACKEND_FAILURE;
    st = exact_gemm_admit(*plan, *A, *B, *C, stream, adm);
    if (st != RNS8_SUCCESS) return st;
  }
  C->device_current = false;
  if (per_tile_kind(plan->desc.bound_kind) && !plan->schedule.entries.empty())
    st = run_gemm_tiled(*ctx, *plan, *A, *B, *C, stream);
  else
    st = run_gemm(*ctx, *plan, *A, *B, *C, ws->splitk, plan->prefix, make_ladder_plane_consts(plan->prefix), stream);
  if (st != RNS8_SUCCESS) return st;
  if (exact_wide(plan->desc.semantics)) {
    st = commit_exact_proof(*C, *A, *B, *plan, adm, stream);
    if (st != RNS8_SUCCESS) return st;
  }
  if (synchronous) {
    st = sync(stream);
    if (st != RNS8_SUCCESS) return st;
  }
  C->device_current = true;
  C->source_version = output_source_version(A->source_version, B->source_version);
  return RNS8_SUCCESS;
}

// rns8_mi355x_gemm_rns_noalloc: the bounded int64/uint64 GEMM of
// rns8_mi355x_gemm_rns_async without a workspace argument. Split-K residues
// go to the library's per-device static scratch (kNoAllocScratchBytes); the
// call allocates nothing, host or device. Exact-wide plans are refused: their
// admission keeps proofs in host memory and may read one back.
rns8_status gemm_rns_noalloc(rns8_context* ctx, const rns8_plan* plan, const rns8_matrix* A, const rns8_matrix* B,
                             rns8_matrix* C, void* stream_arg) {
  if (!ctx || !plan || !A || !B || !C) return RNS8_INVALID_ARGUMENT;
  if (plan->backend != ctx->backend || plan->device_id != ctx->device_id) return RNS8_INVALID_ARGUMENT;
  rns8_status st = check_rns_operands(*ctx, *plan, *A, *B, *C);
  if (st != RNS8_SUCCESS) return st;
  if (plan->desc.semantics != RNS8_BOUNDED_I64 && plan->desc.semantics != RNS8_BOUNDED_U64)
    return RNS8_UNSUPPORTED_BACKEND;
  const bool tiled = per_tile_kind(plan->desc.bound_kind) && !plan->schedule.entries.empty();
  int8_t* scratch = nullptr;
  if (!tiled && plan->splitk_slices > 1) {
    if (choose_gemm_shape(plan->desc.m, plan->desc.n, plan->desc.k, plan->prefix).ws_bytes > kNoAllocScratchBytes)
      return RNS8_WORKSPACE_TOO_SMALL;
    scratch = noalloc_scratch(ctx->device_id);
    if (!scratch) return RNS8_BACKEND_FAILURE;
  }
  const hipStream_t stream = pick_stream(*ctx, stream_arg);
  C->device_current = false;
  st = tiled ? run_gemm_tiled(*ctx, *plan, *A, *B, *C, stream)
             : run_gemm(*ctx, *plan, *A, *B, *C, scratch, plan->prefix, make_ladder_plane_consts(plan->prefix),
                        stream);
  if (st != RNS8_SUCCESS) return st;
  C->device_current = true;
  C->source_version = output_source_version(A->source_version, B->source_version);
  return RNS8_SUCCESS;
}

// Fused native-input GEMM (rns8_mi355x_gemm_native_*_async): bounded plans
// whose output is small enough for the fused path (fused.hip). The plan's
// declared bound covers the result as it does for rns8_gemm_rns, so no
// operand proof is needed; C must be the plan's output matrix.
template <typename T>
rns8_status gemm_native(rns8_context* ctx, const rns8_plan* plan, const T* A, int64_t lda, const T* B, int64_t ldb,
                        rns8_matrix* C, rns8_workspace* ws, void* stream_arg) {
  constexpr bool is_signed = std::is_same<T, int64_t>::value;
  const rns8_semantics sem = is_signed ? RNS8_BOUNDED_I64 : RNS8_BOUNDED_U64;
  if (!ctx || !plan || !A || !B || !C || !ws) return RNS8_INVALID_ARGUMENT;
  if (plan->desc.semantics != sem) return RNS8_INVALID_ARGUMENT;
  rns8_status st = check_plan_ctx_ws(*ctx, *plan, *ws);
  if (st != RNS8_SUCCESS) return st;
  const int64_t m = plan->desc.m, n = plan->desc.n, k = plan->desc.k;
  if (!valid_access(m, k, lda) || !valid_access(k, n, ldb)) return RNS8_INVALID_ARGUMENT;
  if (C->backend != plan->backend || C->device_id != ctx->device_id) return RNS8_INVALID_ARGUMENT;
  if (!matrix_matches(*C, sem, storage_bound_kind(*plan), m, n, storage_prefix(*plan), plan->desc.tile_m,
                      plan->desc.tile_n))
    return RNS8_INVALID_ARGUMENT;
  if (!plan->fused_ok || plan->fused.ws_bytes > ws->splitk_bytes) return RNS8_UNSUPPORTED_BACKEND;
  const hipStream_t stream = pick_stream(*ctx, stream_arg);
  FusedArgs f{};
  f.a = A;
  f.b = B;
  f.lda = lda;
  f.ldb = ldb;
  f.m = m;
  f.n = n;
  f.k = k;
  f.c = C->planes;
  f.ldc = C->plane_ld;
  f.pitch_c = C->plane_pitch;
  f.nplanes = plan->prefix;
  f.kind = is_signed ? NativeKind::I64 : NativeKind::U64;
  f.ws = ws->splitk;
  f.shape = plan->fused;
  // a refused call leaves C as it was
  if (!fused_args_ok(f)) return RNS8_UNSUPPORTED_BACKEND;
  if (hipSetDevice(ctx->device_id) != hipSuccess) return RNS8_BACKEND_FAILURE;
  C->device_current = false;
  const hipError_t e = launch_fused_native(f, make_ladder_plane_consts(plan->prefix), stream);
  if (e == hipErrorInvalidValue) return RNS8_UNSUPPORTED_BACKEND;
  if (e != hipSuccess) return RNS8_BACKEND_FAILURE;
  C->device_current = true;
  C->source_version = 0;  // native device operands carry no source version
  return RNS8_SUCCESS;
}

rns8_status gemm_finite(rns8_context* ctx, const rns8_plan* plan, uint16_t modulus, const rns8_matrix* A,
                        const rns8_matrix* B, rns8_matrix* C, rns8_workspace* ws, void* stream_arg, bool synchronous) {
  if (!ctx || !plan || !A || !B || !C || !ws) return RNS8_INVALID_ARGUMENT;
  rns8_status st = check_plan_ctx_ws(*ctx, *plan, *ws);
  if (st != RNS8_SUCCESS) return st;
  st = check_finite_operands(*ctx, *plan, modulus, *A, *B, *C);
  if (st != RNS8_SUCCESS) return st;
  const hipStream_t stream = pick_stream(*ctx, stream_arg);
  C->device_current = false;
  st = run_gemm(*ctx, *plan, *A, *B, *C, ws->splitk, 1, make_single_plane_consts(modulus), stream);
  if (st != RNS8_SUCCESS) return st;
  if (synchronous) {
    st = sync(stream);
    if (st != RNS8_SUCCESS) return st;
  }
  C->device_current = true;
  C->finite_modulus = modulus;
  C->source_version = output_source_version(A->source_version, B->source_version);
  return RNS8_SUCCESS;
}

// ---- grouped GEMM (reference api_gemm.cpp:200-336, hip_grouped_descriptor.cpp:474-512) ----

// Same-shape resident GEMMs of one plan, each task with its own A, B, C and
// workspace: every task passes the ungrouped checks, no handle appears twice
// in the group, and no result is another task's operand (the tasks run
// concurrently). Global and collapsed per-tile plans run as one persistent
// launch per K block with the task folded into the unit order; per-tile plans
// with a schedule run the listed GEMM per task.
rns8_status gemm_grouped(rns8_context* ctx, const rns8_plan* plan, const rns8_grouped_gemm_task* tasks,
                         uint32_t task_count, bool finite, uint16_t modulus, void* stream_arg, bool synchronous) {
  if (!ctx || !plan) return RNS8_INVALID_ARGUMENT;
  if (finite ? (!uses_finite_storage(plan->desc.semantics) || plan->desc.finite_modulus != modulus ||
                !valid_finite_modulus(plan->desc.semantics, modulus))
             : !uses_rns_storage(plan->desc.semantics))
    return RNS8_INVALID_ARGUMENT;
  if (!tasks || task_count <= 1) return RNS8_INVALID_ARGUMENT;
  for (uint32_t i = 0; i < task_count; ++i) {
    const rns8_grouped_gemm_task& t = tasks[i];
    if (!valid_abi(t.struct_size, t.abi_version, sizeof(t)) || !t.a || !t.b || !t.c || !t.workspace)
      return RNS8_INVALID_ARGUMENT;
    const rns8_status st = check_plan_ctx_ws(*ctx, *plan, *t.workspace);
    if (st != RNS8_SUCCESS) return st;
  }
  for (uint32_t i = 0; i < task_count; ++i) {
    const rns8_grouped_gemm_task& t = tasks[i];
    if (t.a == t.b) return RNS8_INVALID_ARGUMENT;
    for (uint32_t j = 0; j < task_count; ++j) {
      const rns8_grouped_gemm_task& u = tasks[j];
      if (t.c == u.a || t.c == u.b) return RNS8_INVALID_ARGUMENT;
      if (j < i && (t.a == u.a || t.b == u.b || t.c == u.c || t.workspace == u.workspace))
        return RNS8_INVALID_ARGUMENT;
    }
    const rns8_status st = finite ? check_finite_operands(*ctx, *plan, modulus, *t.a, *t.b, *t.c)
                                  : check_rns_operands(*ctx, *plan, *t.a, *t.b, *t.c);
    if (st != RNS8_SUCCESS) return st;
  }
  // every host allocation comes before the first change to a result
  std::vector<ExactAdmission> adms(task_count);
  std::vector<TaskPtrs> ptrs(task_count);
  for (uint32_t i = 0; i < task_count; ++i)
    ptrs[i] = TaskPtrs{tasks[i].a->planes, tasks[i].b->planes, tasks[i].c->planes,
                       plan->splitk_slices > 1 ? tasks[i].workspace->splitk : nullptr};
  const hipStream_t stream = pick_stream(*ctx, stream_arg);
  if (hipSetDevice(ctx->device_id) != hipSuccess) return RNS8_BACKEND_FAILURE;
  // every task is admitted before any result changes (a refined admission
  // writes only its result's free proof set)
  if (!finite && exact_wide(plan->desc.semantics))
    for (uint32_t i = 0; i < task_count; ++i) {
      const rns8_status st = exact_gemm_admit(*plan, *tasks[i].a, *tasks[i].b, *tasks[i].c, stream, adms[i]);
      if (st != RNS8_SUCCESS) return st;
    }
  for (uint32_t i = 0; i < task_count; ++i) tasks[i].c->device_current = false;
  rns8_status st = RNS8_SUCCESS;
  if (!finite && per_tile_kind(plan->desc.bound_kind) && !plan->schedule.entries.empty()) {
    for (uint32_t i = 0; i < task_count && st == RNS8_SUCCESS; ++i)
      st = run_gemm_tiled(*ctx, *plan, *tasks[i].a, *tasks[i].b, *tasks[i].c, stream);
  } else {
    const rns8_matrix& a0 = *tasks[0].a;
    const rns8_matrix& b0 = *tasks[0].b;
    const rns8_matrix& c0 = *tasks[0].c;
    GemmArgs g{};
    g.m = plan->desc.m;
    g.n = plan->desc.n;
    g.k = plan->desc.k;
    g.lda = a0.plane_ld;
    g.ldb = b0.plane_ld;
    g.ldc = c0.plane_ld;
    g.pitch_a = a0.plane_pitch;
    g.pitch_b = b0.plane_pitch;
    g.pitch_c = c0.plane_pitch;
    g.nplanes = finite ? 1u : plan->prefix;
    g.slices = plan->splitk_slices;
    const PlaneConsts consts = finite ? make_single_plane_consts(modulus) : make_ladder_plane_consts(plan->prefix);
    const hipError_t e = launch_gemm_grouped(g, consts, ptrs.data(), task_count, stream);
    st = e == hipSuccess ? RNS8_SUCCESS : e == hipErrorInvalidValue ? RNS8_UNSUPPORTED_BACKEND : RNS8_BACKEND_FAILURE;
  }
  if (st == RNS8_SUCCESS && !finite && exact_wide(plan->desc.semantics))
    for (uint32_t i = 0; i < task_count && st == RNS8_SUCCESS; ++i)
      st = commit_exact_proof(*tasks[i].c, *tasks[i].a, *tasks[i].b, *plan, adms[i], stream);
  if (st == RNS8_SUCCESS && synchronous) st = sync(stream);
  if (st != RNS8_SUCCESS) return st;
  for (uint32_t i = 0; i < task_count; ++i) {
    rns8_matrix& C = *tasks[i].c;
    C.device_current = true;
    C.source_version = output_source_version(tasks[i].a->source_version, tasks[i].b->source_version);
    if (finite) C.finite_modulus = modulus;
  }
  return RNS8_SUCCESS;
}

// ---- export ------------------------------------------------------------------------

struct ExportRequest {
  ExportKind kind;
  rns8_semantics semantics;
  uint32_t limbs;
};

// Global plans: one launch at the plan prefix. Per-tile plans: one launch per
// prefix group of tiles, each tile with its own bound, and one for the
// zero-output tiles (reference api_export.cpp:365-410).
hipError_t launch_plan_export(const rns8_plan& plan, const ExportArgs& a, hipStream_t stream) {
  if (!per_tile_kind(plan.desc.bound_kind)) return launch_export(a, plan.prefix, stream);
  for (const auto& g : plan.export_groups) {
    const TileExport* const t = plan.export_tiles + g.first;
    const hipError_t e =
        g.prefix == 0 ? launch_export_zero_tiles(a, t, g.count, plan.desc.tile_m, plan.desc.tile_n, stream)
                      : launch_export_tiles(a, g.prefix, t, g.count, plan.desc.tile_m, plan.desc.tile_n, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// Host export: reconstruct into a compact device staging buffer, read the
// status word, and copy to `dst` only when every cell is in range, so a
// RANGE_ERROR leaves the caller's buffer untouched (api_export.cpp:365-414,
// hip_backend_export_bounded.inc:55-67).
rns8_status export_host(rns8_context* ctx, const rns8_plan* plan, const rns8_matrix* C, void* dst, int64_t ld,
                        const ExportRequest& req) {
  rns8_status st = check_export(*ctx, *plan, *C, req.semantics);
  if (st != RNS8_SUCCESS) return st;
  auto* mc = const_cast<rns8_matrix*>(C);
  const int64_t m = plan->desc.m, n = plan->desc.n;
  const std::size_t elem = sizeof(uint64_t) * req.limbs;
  const std::size_t bytes = static_cast<std::size_t>(m) * n * elem;
  if (hipSetDevice(ctx->device_id) != hipSuccess) return RNS8_BACKEND_FAILURE;
  st = ensure_device_buffer(ctx->device_id, &mc->staging, &mc->staging_bytes, bytes);
  if (st != RNS8_SUCCESS) return st;
  if (!mc->status && hipMalloc(reinterpret_cast<void**>(&mc->status), 64) != hipSuccess) return RNS8_BACKEND_FAILURE;
  const hipStream_t stream = ctx->stream;
  if (launch_zero_words(mc->status, 1, stream) != hipSuccess) return RNS8_BACKEND_FAILURE;
  const ExportArgs a = export_args(*plan, *C, mc->staging, n, req.limbs, req.kind, mc->status);
  if (launch_plan_export(*plan, a, stream) != hipSuccess) return RNS8_BACKEND_FAILURE;
  uint32_t status = 0;
  if (hipMemcpyAsync(&status, mc->status, sizeof(status), hipMemcpyDeviceToHost, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return RNS8_BACKEND_FAILURE;
  if (status != 0) return RNS8_RANGE_ERROR;
  if (ctx->host.to_host(dst, ld * elem, mc->staging, n * elem, m, stream) != hipSuccess) return RNS8_BACKEND_FAILURE;
  return RNS8_SUCCESS;
}

rns8_status export_device(rns8_context* ctx, const rns8_plan* plan, const rns8_matrix* C, void* d_dst, int64_t ld,
                          uint32_t* d_status, void* stream_arg, const ExportRequest& req) {
  if (!d_status) return RNS8_INVALID_ARGUMENT;
  rns8_status st = check_export(*ctx, *plan, *C, req.semantics);
  if (st != RNS8_SUCCESS) return st;
  if (hipSetDevice(ctx->device_id) != hipSuccess) return RNS8_BACKEND_FAILURE;
  const ExportArgs a = export_args(*plan, *C, d_dst, ld, req.limbs, req.kind, d_status);
  return launch_plan_export(*plan, a, pick_stream(*ctx, stream_arg)) == hipSuccess
             ? RNS8_SUCCESS
             : RNS8_BACKEND_FAILURE;
}

rns8_status export_finite(rns8_context* ctx, const rns8_plan* plan, uint16_t modulus, const rns8_matrix* C,
                          uint8_t* dst, int64_t ld, Source where, void* stream_arg) {
  if (!ctx || !plan || !C || !dst || !valid_access(plan->desc.m, plan->desc.n, ld)) return RNS8_INVALID_ARGUMENT;
  rns8_status st = check_finite_export(*ctx, *plan, modulus, *C);
  if (st != RNS8_SUCCESS) return st;
  auto* mc = const_cast<rns8_matrix*>(C);
  const int64_t m = plan->desc.m, n = plan->desc.n;
  if (hipSetDevice(ctx->device_id) != hipSuccess) return RNS8_BACKEND_FAILURE;
  const hipStream_t stream = pick_stream(*ctx, stream_arg);
  if (where == Source::Device) {
    const ExportU8Args a = export_u8_args(*plan, *C, dst, ld, modulus);
    return launch_export_u8(a, stream) == hipSuccess ? RNS8_SUCCESS : RNS8_BACKEND_FAILURE;
  }
  st = ensure_device_buffer(ctx->device_id, &mc->staging, &mc->staging_bytes, static_cast<std::size_t>(m) * n);
  if (st != RNS8_SUCCESS) return st;
  const ExportU8Args a = export_u8_args(*plan, *C, static_cast<uint8_t*>(mc->staging), n, modulus);
  if (launch_export_u8(a, stream) != hipSuccess) return RNS8_BACKEND_FAILURE;
  return ctx->host.to_host(dst, ld, mc->staging, n, m, stream) == hipSuccess ? RNS8_SUCCESS : RNS8_BACKEND_FAILURE;
}

// ---- one-shot (api_oneshot.cpp) -----------------------------------------------------

struct OneshotState {
  rns8_plan* plan = nullptr;
  rns8_matrix* A = nullptr;
  rns8_matrix* B = nullptr;
  rns8_matrix* C = nullptr;
  rns8_workspace* ws = nullptr;
  ~OneshotState() {
    rns8_destroy_workspace(ws);
    rns8_destroy_matrix(C);
    rns8_destroy_matrix(B);
    rns8_destroy_matrix(A);
    rns8_destroy_plan(plan);
  }
};

rns8_matrix_desc make_matrix_desc(int64_t rows, int64_t cols, rns8_semantics s, rns8_bound_kind bk, uint32_t prefix,
                                  uint32_t tile_m, uint32_t tile_n) {
  rns8_matrix_desc d{};
  d.struct_size = sizeof(d);
  d.abi_version = RNS8_ABI_VERSION;
  d.rows = rows;
  d.cols = cols;
  d.logical_ld = cols;
  d.semantics = s;
  d.logical_layout = RNS8_LAYOUT_ROW_MAJOR;
  d.bound_kind = bk;
  d.tile_m = tile_m;
  d.tile_n = tile_n;
  d.max_prefix = prefix;
  return d;
}

}  // namespace

// The last oneshot call's device state. The reference creates and destroys
// the plan, matrices and workspace on every call (api_oneshot.cpp:107-133);
// here an equal descriptor on the same context reuses them, which removes the
// allocations (~2.5 ms at 4096^3) from repeated calls. Descriptors with
// per-tile bound arrays or proof masks are not cached.
struct OneshotCache {
  rns8_gemm_desc desc{};
  bool reusable = false;  // false: freed when its call returns
  OneshotState state;
};

void release_oneshot_cache(rns8_context& ctx) {
  delete ctx.oneshot;
  ctx.oneshot = nullptr;
}

namespace {

bool same_oneshot_desc(const rns8_gemm_desc& a, const rns8_gemm_desc& b) {
  return a.struct_size == b.struct_size && a.abi_version == b.abi_version && a.semantics == b.semantics &&
         a.bound_kind == b.bound_kind && a.requested_backend == b.requested_backend && a.m == b.m && a.n == b.n &&
         a.k == b.k && a.bound == b.bound && a.max_prefix == b.max_prefix && a.tile_m == b.tile_m &&
         a.tile_n == b.tile_n && a.finite_modulus == b.finite_modulus && a.flags == b.flags &&
         a.lhs_bound == b.lhs_bound && a.rhs_bound == b.rhs_bound;
}

bool cacheable_oneshot_desc(const rns8_gemm_desc& d) {
  return !d.tile_bounds && d.tile_bounds_count == 0 && !d.zero_a_rows && d.zero_a_rows_count == 0 &&
         !d.zero_b_cols && d.zero_b_cols_count == 0;
}

rns8_status create_oneshot(rns8_context* ctx, const rns8_gemm_desc& desc, OneshotState& s) {
  rns8_status st = rns8_create_plan(ctx, &desc, &s.plan);
  if (st != RNS8_SUCCESS) return st;
  const rns8_bound_kind bk = storage_bound_kind(*s.plan);
  const uint32_t sp = storage_prefix(*s.plan);
  const uint32_t tm = s.plan->desc.tile_m, tn = s.plan->desc.tile_n;
  const rns8_matrix_desc ad = make_matrix_desc(desc.m, desc.k, desc.semantics, bk, sp, tm, tn);
  const rns8_matrix_desc bd = make_matrix_desc(desc.k, desc.n, desc.semantics, bk, sp, tm, tn);
  const rns8_matrix_desc cd = make_matrix_desc(desc.m, desc.n, desc.semantics, bk, sp, tm, tn);
  st = rns8_create_matrix(ctx, &ad, &s.A);
  if (st == RNS8_SUCCESS) st = rns8_create_matrix(ctx, &bd, &s.B);
  if (st == RNS8_SUCCESS) st = rns8_create_matrix(ctx, &cd, &s.C);
  if (st == RNS8_SUCCESS) st = rns8_create_workspace(ctx, s.plan, &s.ws);
  return st;
}

// The state for a oneshot call: the cached one when the descriptor matches,
// else a new one that replaces the cache. Matrices are packed with source
// version 0 (never elided), so stale residues are never reused.
rns8_status oneshot_state(rns8_context* ctx, const rns8_gemm_desc& desc, OneshotState*& out) {
  out = nullptr;
  if (ctx->oneshot && ctx->oneshot->reusable && same_oneshot_desc(ctx->oneshot->desc, desc)) {
    out = &ctx->oneshot->state;
    return RNS8_SUCCESS;
  }
  release_oneshot_cache(*ctx);
  auto* cache = new (std::nothrow) OneshotCache();
  if (!cache) return RNS8_INTERNAL_ERROR;
  const rns8_status st = create_oneshot(ctx, desc, cache->state);
  if (st != RNS8_SUCCESS) {
    delete cache;
    return st;
  }
  cache->desc = desc;
  cache->desc.tile_bounds = nullptr;
  cache->desc.zero_a_rows = nullptr;
  cache->desc.zero_b_cols = nullptr;
  cache->reusable = cacheable_oneshot_desc(desc);
  ctx->oneshot = cache;
  out = &cache->state;
  return RNS8_SUCCESS;
}

// A oneshot call that ends in an exception (an allocation failure, caught at
// the API boundary) keeps no cached state either.
struct KeepOneshotOnSuccess {
  rns8_context* ctx;
  ~KeepOneshotOnSuccess() {
    if (std::uncaught_exceptions() > 0) release_oneshot_cache(*ctx);
  }
};

// reference api_oneshot.cpp:440-466
rns8_status typed_oneshot_contract(const rns8_context& ctx, const rns8_gemm_desc& desc, rns8_semantics expected,
                                   int64_t lda, int64_t ldb, int64_t ldc) {
  if (!valid_abi(desc.struct_size, desc.abi_version, sizeof(desc)) || desc.semantics != expected)
    return RNS8_INVALID_ARGUMENT;
  const uint32_t budget = desc.max_prefix == 0 ? default_prefix(desc.semantics) : desc.max_prefix;
  const rns8_status v = validate_gemm_desc(desc, budget);
  if (v != RNS8_SUCCESS) return v;
  if (!valid_access(desc.m, desc.k, lda) || !valid_access(desc.k, desc.n, ldb) || !valid_access(desc.m, desc.n, ldc))
    return RNS8_INVALID_ARGUMENT;
  if (desc.requested_backend != RNS8_BACKEND_AUTO && desc.requested_backend != ctx.backend)
    return RNS8_UNSUPPORTED_BACKEND;
  return RNS8_SUCCESS;
}

// reference api_oneshot.cpp:78-106
rns8_status finite_oneshot_contract(const rns8_context& ctx, const rns8_gemm_desc& desc, rns8_semantics expected,
                                    uint16_t modulus, int64_t lda, int64_t ldb, int64_t ldc) {
  if (!valid_abi(desc.struct_size, desc.abi_version, sizeof(desc)) || desc.semantics != expected)
    return RNS8_INVALID_ARGUMENT;
  const bool tiles_ok = (desc.tile_m == 0 || (desc.tile_m >= 64 && desc.tile_m <= 512 && !(desc.tile_m & (desc.tile_m - 1)))) &&
                        (desc.tile_n == 0 || (desc.tile_n >= 64 && desc.tile_n <= 512 && !(desc.tile_n & (desc.tile_n - 1))));
  if (!valid_finite_modulus(expected, modulus) || desc.m <= 0 || desc.n <= 0 || desc.k <= 0 ||
      desc.bound_kind != RNS8_BOUND_NONE || desc.bound != 0 || desc.max_prefix != 0 || desc.finite_modulus != modulus ||
      desc.flags != 0 || desc.tile_bounds || desc.tile_bounds_count != 0 || desc.lhs_bound != 0 ||
      desc.rhs_bound != 0 || !tiles_ok)
    return RNS8_INVALID_ARGUMENT;
  if (!valid_access(desc.m, desc.k, lda) || !valid_access(desc.k, desc.n, ldb) || !valid_access(desc.m, desc.n, ldc))
    return RNS8_INVALID_ARGUMENT;
  if (desc.requested_backend != RNS8_BACKEND_AUTO && desc.requested_backend != ctx.backend)
    return RNS8_UNSUPPORTED_BACKEND;
  return RNS8_SUCCESS;
}

template <typename T>
rns8_status bounded_oneshot(rns8_context* ctx, const rns8_gemm_desc* desc, const T* A, int64_t lda, const T* B,
                            int64_t ldb, T* C, int64_t ldc) {
  constexpr bool is_signed = std::is_same<T, int64_t>::value;
  if (!ctx || !desc || !A || !B || !C) return RNS8_INVALID_ARGUMENT;
  const rns8_status pre =
      typed_oneshot_contract(*ctx, *desc, is_signed ? RNS8_BOUNDED_I64 : RNS8_BOUNDED_U64, lda, ldb, ldc);
  if (pre != RNS8_SUCCESS) return pre;
  OneshotState* sp = nullptr;
  rns8_status st = oneshot_state(ctx, *desc, sp);
  if (st != RNS8_SUCCESS) return st;
  const KeepOneshotOnSuccess keep{ctx};
  OneshotState& s = *sp;
  st = pack_native<T>(ctx, s.A, A, lda, 0, Source::Host, nullptr);
  if (st == RNS8_SUCCESS) st = pack_native<T>(ctx, s.B, B, ldb, 0, Source::Host, nullptr);
  if (st == RNS8_SUCCESS) st = gemm_rns(ctx, s.plan, s.A, s.B, s.C, s.ws, nullptr, true);
  if (st == RNS8_SUCCESS) {
    if (!valid_access(s.plan->desc.m, s.plan->desc.n, ldc)) st = RNS8_INVALID_ARGUMENT;
    else
      st = export_host(ctx, s.plan, s.C, C, ldc,
                       ExportRequest{is_signed ? ExportKind::I64 : ExportKind::U64,
                                     is_signed ? RNS8_BOUNDED_I64 : RNS8_BOUNDED_U64, 1});
  }
  // a failed call, or one whose descriptor is not cacheable, keeps nothing
  if (st != RNS8_SUCCESS || !ctx->oneshot->reusable) release_oneshot_cache(*ctx);
  return st;
}

rns8_status finite_oneshot(rns8_context* ctx, const rns8_gemm_desc* desc, rns8_semantics sem, uint16_t modulus,
                           const uint8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, uint8_t* C, int64_t ldc) {
  if (!ctx || !desc || !A || !B || !C) return RNS8_INVALID_ARGUMENT;
  const rns8_status pre = finite_oneshot_contract(*ctx, *desc, sem, modulus, lda, ldb, ldc);
  if (pre != RNS8_SUCCESS) return pre;
  OneshotState* sp = nullptr;
  rns8_status st = oneshot_state(ctx, *desc, sp);
  if (st != RNS8_SUCCESS) return st;
  const KeepOneshotOnSuccess keep{ctx};
  OneshotState& s = *sp;
  st = pack_u8(ctx, s.A, modulus, A, lda, 0, Source::Host, nullptr);
  if (st == RNS8_SUCCESS) st = pack_u8(ctx, s.B, modulus, B, ldb, 0, Source::Host, nullptr);
  if (st == RNS8_SUCCESS) st = gemm_finite(ctx, s.plan, modulus, s.A, s.B, s.C, s.ws, nullptr, true);
  if (st == RNS8_SUCCESS) st = export_finite(ctx, s.plan, modulus, s.C, C, ldc, Source::Host, nullptr);
  if (st != RNS8_SUCCESS || !ctx->oneshot->reusable) release_oneshot_cache(*ctx);
  return st;
}

}  // namespace
}  // namespace rns8x

using namespace rns8x;

// ---- public ABI ------------------------------------------------------------------------

rns8_status rns8_pack_i64(rns8_context* ctx, rns8_matrix* matrix, const int64_t* src, int64_t ld,
                          uint64_t source_version) {
  return guard([&] { return pack_native<int64_t>(ctx, matrix, src, ld, source_version, Source::Host, nullptr); });
}

rns8_status rns8_pack_u64(rns8_context* ctx, rns8_matrix* matrix, const uint64_t* src, int64_t ld,
                          uint64_t source_version) {
  return guard([&] { return pack_native<uint64_t>(ctx, matrix, src, ld, source_version, Source::Host, nullptr); });
}

rns8_status rns8_pack_finite_u8(rns8_context* ctx, rns8_matrix* matrix, uint16_t modulus, const uint8_t* src,
                                int64_t ld, uint64_t source_version) {
  return guard([&] { return pack_u8(ctx, matrix, modulus, src, ld, source_version, Source::Host, nullptr); });
}

rns8_status rns8_gemm_rns(rns8_context* ctx, const rns8_plan* plan, const rns8_matrix* A, const rns8_matrix* B,
                          rns8_matrix* C, rns8_workspace* workspace) {
  return guard([&] { return gemm_rns(ctx, plan, A, B, C, workspace, nullptr, true); });
}

rns8_status rns8_gemm_finite_u8(rns8_context* ctx, const rns8_plan* plan, uint16_t modulus, const rns8_matrix* A,
                                const rns8_matrix* B, rns8_matrix* C, rns8_workspace* workspace) {
  return guard([&] { return gemm_finite(ctx, plan, modulus, A, B, C, workspace, nullptr, true); });
}

rns8_status rns8_export_i64(rns8_context* ctx, const rns8_plan* plan, const rns8_matrix* C, int64_t* dst, int64_t ld) {
  return guard([&]() -> rns8_status {
    if (!ctx || !plan || !C || !dst || !valid_access(plan->desc.m, plan->desc.n, ld)) return RNS8_INVALID_ARGUMENT;
    return export_host(ctx, plan, C, dst, ld, ExportRequest{ExportKind::I64, RNS8_BOUNDED_I64, 1});
  });
}

rns8_status rns8_export_u64(rns8_context* ctx, const rns8_plan* plan, const rns8_matrix* C, uint64_t* dst,
                            int64_t ld) {
  return guard([&]() -> rns8_status {
    if (!ctx || !plan || !C || !dst || !valid_access(plan->desc.m, plan->desc.n, ld)) return RNS8_INVALID_ARGUMENT;
    return export_host(ctx, plan, C, dst, ld, ExportRequest{ExportKind::U64, RNS8_BOUNDED_U64, 1});
  });
}

rns8_status rns8_export_exact_wide_signed_limbs(rns8_context* ctx, const rns8_plan* plan, const rns8_matrix* C,
                                                uint64_t* dst, int64_t ld, uint32_t limb_count) {
  return guard([&]() -> rns8_status {
    if (!ctx || !plan || !C || !dst || !valid_limb_access(plan->desc.m, plan->desc.n, ld, limb_count))
      return RNS8_INVALID_ARGUMENT;
    return export_host(ctx, plan, C, dst, ld,
                       ExportRequest{ExportKind::WIDE_SIGNED, RNS8_EXACT_WIDE_SIGNED, limb_count});
  });
}

rns8_status rns8_export_exact_wide_unsigned_limbs(rns8_context* ctx, const rns8_plan* plan, const rns8_matrix* C,
                                                  uint64_t* dst, int64_t ld, uint32_t limb_count) {
  return guard([&]() -> rns8_status {
    if (!ctx || !plan || !C || !dst || !valid_limb_access(plan->desc.m, plan->desc.n, ld, limb_count))
      return RNS8_INVALID_ARGUMENT;
    return export_host(ctx, plan, C, dst, ld,
                       ExportRequest{ExportKind::WIDE_UNSIGNED, RNS8_EXACT_WIDE_UNSIGNED, limb_count});
  });
}

rns8_status rns8_export_finite_u8(rns8_context* ctx, const rns8_plan* plan, uint16_t modulus, const rns8_matrix* C,
                                  uint8_t* dst, int64_t ld) {
  return guard([&] { return export_finite(ctx, plan, modulus, C, dst, ld, Source::Host, nullptr); });
}

rns8_status rns8_gemm_rns_grouped(rns8_context* ctx, const rns8_plan* plan, const rns8_grouped_gemm_task* tasks,
                                  uint32_t task_count) {
  return guard([&] { return gemm_grouped(ctx, plan, tasks, task_count, false, 0, nullptr, true); });
}

rns8_status rns8_gemm_finite_u8_grouped(rns8_context* ctx, const rns8_plan* plan, uint16_t modulus,
                                        const rns8_grouped_gemm_task* tasks, uint32_t task_count) {
  return guard([&] { return gemm_grouped(ctx, plan, tasks, task_count, true, modulus, nullptr, true); });
}

rns8_status rns8_gemm_i64_oneshot(rns8_context* ctx, const rns8_gemm_desc* desc, const int64_t* A, int64_t lda,
                                  const int64_t* B, int64_t ldb, int64_t* C, int64_t ldc) {
  return guard([&] { return bounded_oneshot<int64_t>(ctx, desc, A, lda, B, ldb, C, ldc); });
}

rns8_status rns8_gemm_u64_oneshot(rns8_context* ctx, const rns8_gemm_desc* desc, const uint64_t* A, int64_t lda,
                                  const uint64_t* B, int64_t ldb, uint64_t* C, int64_t ldc) {
  return guard([&] { return bounded_oneshot<uint64_t>(ctx, desc, A, lda, B, ldb, C, ldc); });
}

rns8_status rns8_gemm_finite_ring_u8_oneshot(rns8_context* ctx, const rns8_gemm_desc* desc, uint16_t modulus,
                                             const uint8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, uint8_t* C,
                                             int64_t ldc) {
  return guard(
      [&] { return finite_oneshot(ctx, desc, RNS8_FINITE_RING_U8, modulus, A, lda, B, ldb, C, ldc); });
}

rns8_status rns8_gemm_finite_field_u8_oneshot(rns8_context* ctx, const rns8_gemm_desc* desc, uint16_t modulus,
                                              const uint8_t* A, int64_t lda, const uint8_t* B, int64_t ldb,
                                              uint8_t* C, int64_t ldc) {
  return guard(
      [&] { return finite_oneshot(ctx, desc, RNS8_FINITE_FIELD_U8, modulus, A, lda, B, ldb, C, ldc); });
}

// ---- MI355X device-resident extensions ------------------------------------------------

rns8_status rns8_mi355x_pack_i64_device(rns8_context* ctx, rns8_matrix* matrix, const int64_t* d_src, int64_t ld,
                                        uint64_t source_version, void* stream) {
  return guard([&] { return pack_native<int64_t>(ctx, matrix, d_src, ld, source_version, Source::Device, stream); });
}

rns8_status rns8_mi355x_pack_u64_device(rns8_context* ctx, rns8_matrix* matrix, const uint64_t* d_src, int64_t ld,
                                        uint64_t source_version, void* stream) {
  return guard([&] { return pack_native<uint64_t>(ctx, matrix, d_src, ld, source_version, Source::Device, stream); });
}

rns8_status rns8_mi355x_pack_finite_u8_device(rns8_context* ctx, rns8_matrix* matrix, uint16_t modulus,
                                              const uint8_t* d_src, int64_t ld, uint64_t source_version,
                                              void* stream) {
  return guard([&] { return pack_u8(ctx, matrix, modulus, d_src, ld, source_version, Source::Device, stream); });
}

rns8_status rns8_mi355x_gemm_rns_async(rns8_context* ctx, const rns8_plan* plan, const rns8_matrix* A,
                                       const rns8_matrix* B, rns8_matrix* C, rns8_workspace* workspace,
                                       void* stream) {
  return guard([&] { return gemm_rns(ctx, plan, A, B, C, workspace, stream, false); });
}

rns8_status rns8_mi355x_gemm_rns_noalloc(rns8_context* ctx, const rns8_plan* plan, const rns8_matrix* A,
                                         const rns8_matrix* B, rns8_matrix* C, void* stream) {
  return guard([&] { return gemm_rns_noalloc(ctx, plan, A, B, C, stream); });
}

rns8_status rns8_mi355x_gemm_finite_u8_async(rns8_context* ctx, const rns8_plan* plan, uint16_t modulus,
                                             const rns8_matrix* A, const rns8_matrix* B, rns8_matrix* C,
                                             rns8_workspace* workspace, void* stream) {
  return guard([&] { return gemm_finite(ctx, plan, modulus, A, B, C, workspace, stream, false); });
}

rns8_status rns8_mi355x_gemm_native_i64_async(rns8_context* ctx, const rns8_plan* plan, const int64_t* d_A,
                                              int64_t lda, const int64_t* d_B, int64_t ldb, rns8_matrix* C,
                                              rns8_workspace* workspace, void* stream) {
  return guard([&] { return gemm_native<int64_t>(ctx, plan, d_A, lda, d_B, ldb, C, workspace, stream); });
}

rns8_status rns8_mi355x_gemm_native_u64_async(rns8_context* ctx, const rns8_plan* plan, const uint64_t* d_A,
                                              int64_t lda, const uint64_t* d_B, int64_t ldb, rns8_matrix* C,
                                              rns8_workspace* workspace, void* stream) {
  return guard([&] { return gemm_native<uint64_t>(ctx, plan, d_A, lda, d_B, ldb, C, workspace, stream); });
}

rns8_status rns8_mi355x_gemm_rns_grouped_async(rns8_context* ctx, const rns8_plan* plan,
                                              const rns8_grouped_gemm_task* tasks, uint32_t task_count,
                                              void* stream) {
  return guard([&] { return gemm_grouped(ctx, plan, tasks, task_count, false, 0, stream, false); });
}

rns8_status rns8_mi355x_gemm_finite_u8_grouped_async(rns8_context* ctx, const rns8_plan* plan, uint16_t modulus,
                                                    const rns8_grouped_gemm_task* tasks, uint32_t task_count,
                                                    void* stream) {
  return guard([&] { return gemm_grouped(ctx, plan, tasks, task_count, true, modulus, stream, false); });
}

rns8_status rns8_mi355x_export_i64_device(rns8_context* ctx, const rns8_plan* plan, const rns8_matrix* C,
                                          int64_t* d_dst, int64_t ld, uint32_t* d_status, void* stream) {
  return guard([&]() -> rns8_status {
    if (!ctx || !plan || !C || !d_dst || !valid_access(plan->desc.m, plan->desc.n, ld)) return RNS8_INVALID_ARGUMENT;
    return export_device(ctx, plan, C, d_dst, ld, d_status, stream,
                         ExportRequest{ExportKind::I64, RNS8_BOUNDED_I64, 1});
  });
}

rns8_status rns8_mi355x_export_u64_device(rns8_context* ctx, const rns8_plan* plan, const rns8_matrix* C,
                                          uint64_t* d_dst, int64_t ld, uint32_t* d_status, void* stream) {
  return guard([&]() -> rns8_status {
    if (!ctx || !plan || !C || !d_dst || !valid_access(plan->desc.m, plan->desc.n, ld)) return RNS8_INVALID_ARGUMENT;
    return export_device(ctx, plan, C, d_dst, ld, d_status, stream,
                         ExportRequest{ExportKind::U64, RNS8_BOUNDED_U64, 1});
  });
}

rns8_status rns8_mi355x_export_exact_wide_signed_limbs_device(rns8_context* ctx, const rns8_plan* plan,
                                                              const rns8_matrix* C, uint64_t* d_dst, int64_t ld,
                                                              uint32_t limb_count, uint32_t* d_status, void* stream) {
  return guard([&]() -> rns8_status {
    if (!ctx || !plan || !C || !d_dst || !valid_limb_access(plan->desc.m, plan->desc.n, ld, limb_count))
      return RNS8_INVALID_ARGUMENT;
    return export_device(ctx, plan, C, d_dst, ld, d_status, stream,
                         ExportRequest{ExportKind::WIDE_SIGNED, RNS8_EXACT_WIDE_SIGNED, limb_count});
  });
}

rns8_status rns8_mi355x_export_exact_wide_unsigned_limbs_device(rns8_context* ctx, const rns8_plan* plan,
                                                                const rns8_matrix* C, uint64_t* d_dst, int64_t ld,
                                                                uint32_t limb_count, uint32_t* d_status,
                                                                void* stream) {
  return guard([&]() -> rns8_status {
    if (!ctx || !plan || !C || !d_dst || !valid_limb_access(plan->desc.m, plan->desc.n, ld, limb_count))
      return RNS8_INVALID_ARGUMENT;
    return export_device(ctx, plan, C, d_dst, ld, d_status, stream,
                         ExportRequest{ExportKind::WIDE_UNSIGNED, RNS8_EXACT_WIDE_UNSIGNED, limb_count});
  });
}

rns8_status rns8_mi355x_export_finite_u8_device(rns8_context* ctx, const rns8_plan* plan, uint16_t modulus,
                                                const rns8_matrix* C, uint8_t* d_dst, int64_t ld, void* stream) {
  return guard([&] { return export_finite(ctx, plan, modulus, C, d_dst, ld, Source::Device, stream); });
}

static_assert(sizeof(rns8_mi355x_exact_axis) == sizeof(rns8x::xa::AxisRecord), "proof record layout");

rns8_status rns8_mi355x_get_exact_proof(rns8_context* ctx, const rns8_matrix* matrix, uint64_t bound[4],
                                        uint32_t* axes_kind, rns8_mi355x_exact_axis* rows,
                                        rns8_mi355x_exact_axis* cols) {
  return guard([&]() -> rns8_status {
    if (!ctx || !matrix || !bound || !axes_kind) return RNS8_INVALID_ARGUMENT;
    if (!exact_wide(matrix->desc.semantics) || matrix->exact_prefix == 0 || matrix->device_id != ctx->device_id)
      return RNS8_INVALID_ARGUMENT;
    if (hipSetDevice(ctx->device_id) != hipSuccess) return RNS8_BACKEND_FAILURE;
    if (matrix->proof_kind == rns8_matrix::ProofKind::Lazy) {
      if (hipStreamWaitEvent(ctx->stream, matrix->proof_event, 0) != hipSuccess) return RNS8_BACKEND_FAILURE;
      const rns8_status st = materialize_proof(*matrix, ctx->stream);
      if (st != RNS8_SUCCESS) return st;
    }
    if (hipEventSynchronize(matrix->proof_event) != hipSuccess) return RNS8_BACKEND_FAILURE;
    const uint32_t s = matrix->proof_set;
    const rns8_matrix::ProofKind kind = matrix->proof_kind;
    *axes_kind = kind == rns8_matrix::ProofKind::Native    ? RNS8_MI355X_EXACT_AXES_NATIVE
                 : kind == rns8_matrix::ProofKind::Carried ? RNS8_MI355X_EXACT_AXES_CARRIED
                                                           : RNS8_MI355X_EXACT_AXES_NONE;
    if (hipMemcpy(bound, matrix->proof_words(s), 4 * sizeof(uint64_t), hipMemcpyDeviceToHost) != hipSuccess)
      return RNS8_BACKEND_FAILURE;
    if (*axes_kind != RNS8_MI355X_EXACT_AXES_NONE) {
      const std::size_t rb = static_cast<std::size_t>(matrix->desc.rows) * sizeof(rns8_mi355x_exact_axis);
      const std::size_t cb = static_cast<std::size_t>(matrix->desc.cols) * sizeof(rns8_mi355x_exact_axis);
      if ((rows && hipMemcpy(rows, matrix->proof_rows(s), rb, hipMemcpyDeviceToHost) != hipSuccess) ||
          (cols && hipMemcpy(cols, matrix->proof_cols(s), cb, hipMemcpyDeviceToHost) != hipSuccess))
        return RNS8_BACKEND_FAILURE;
    }
    I512 b;
    for (int i = 0; i < 4; ++i) b.w[i] = bound[i];
    matrix->exact_max = b;
    matrix->exact_pending = false;
    return RNS8_SUCCESS;
  });
}
