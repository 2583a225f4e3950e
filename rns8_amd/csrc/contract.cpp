// The host-side contract of pack -> GEMM -> export (contract.hpp): argument
// checks of the ABI calls, the kernel arguments of a validated call and the
// launchers' checks of them. Statuses and their order follow the reference:
//   rns8_pack_*          src/core/api_pack.cpp:31-76
//   rns8_gemm_rns        src/core/api_gemm.cpp:50-111
//   rns8_gemm_finite_u8  src/core/api_gemm.cpp:113-160
//   rns8_export_*        src/core/api_export.cpp:5-53
//   rns8_create_matrix   src/core/moduli.cpp:389-448, api_matrix_public_api.inc:84-104
#include "contract.hpp"

#include "exact_proof.hpp"

#include <limits>

namespace rns8x {

bool valid_access(int64_t rows, int64_t cols, int64_t ld) {
  if (rows <= 0 || cols <= 0 || ld < cols) return false;
  return rows <= std::numeric_limits<int64_t>::max() / ld;
}

bool valid_limb_access(int64_t rows, int64_t cols, int64_t ld, uint32_t limbs) {
  if (!valid_access(rows, cols, ld) || limbs == 0 || limbs > 32) return false;
  const int64_t max = std::numeric_limits<int64_t>::max();
  if (ld > max / static_cast<int64_t>(limbs)) return false;
  return rows <= max / (ld * static_cast<int64_t>(limbs));
}

rns8_status init_matrix(const rns8_matrix_desc& d, rns8_backend_kind backend, int device_id, rns8_matrix& m) {
  if (!valid_abi(d.struct_size, d.abi_version, sizeof(d))) return RNS8_INVALID_ARGUMENT;
  const uint32_t prefix = d.max_prefix == 0 ? default_prefix(d.semantics) : d.max_prefix;
  const rns8_status v = validate_matrix_desc(d, prefix);
  if (v != RNS8_SUCCESS) return v;
  if (d.semantics == RNS8_WRAP_U64_MOD_2_64) return RNS8_UNSUPPORTED_BACKEND;
  const int64_t pitch = plane_pitch(d.rows, d.cols);
  const uint32_t planes = uses_finite_storage(d.semantics) ? 1u : prefix;
  if (pitch <= 0 || static_cast<uint64_t>(pitch) > std::numeric_limits<uint64_t>::max() / planes)
    return RNS8_RANGE_ERROR;
  m.desc = d;
  m.desc.max_prefix = uses_finite_storage(d.semantics) ? 0u : prefix;
  if (m.desc.logical_ld == 0) m.desc.logical_ld = m.desc.cols;
  if (m.desc.tile_m == 0) m.desc.tile_m = 128;
  if (m.desc.tile_n == 0) m.desc.tile_n = 128;
  m.backend = backend;
  m.device_id = device_id;
  m.prefix = planes;
  m.plane_ld = padded_ld(d.cols);
  m.plane_pitch = pitch;
  m.plane_bytes = static_cast<uint64_t>(pitch) * planes;
  return RNS8_SUCCESS;
}

rns8_status check_plan_ctx_ws(const rns8_context& ctx, const rns8_plan& plan, const rns8_workspace& ws) {
  if (plan.backend != ctx.backend || ws.backend != plan.backend) return RNS8_INVALID_ARGUMENT;
  if (ws.semantics != plan.desc.semantics || ws.bound_kind != plan.desc.bound_kind) return RNS8_INVALID_ARGUMENT;
  if (ws.m != plan.desc.m || ws.n != plan.desc.n || ws.k != plan.desc.k || ws.prefix != plan.prefix)
    return RNS8_WORKSPACE_TOO_SMALL;
  if (plan.splitk_bytes > ws.splitk_bytes) return RNS8_WORKSPACE_TOO_SMALL;
  if (plan.device_id != ctx.device_id || ws.device_id != ctx.device_id) return RNS8_INVALID_ARGUMENT;
  return RNS8_SUCCESS;
}

// reference api_gemm.cpp:50-111
rns8_status check_rns_operands(const rns8_context& ctx, const rns8_plan& plan, const rns8_matrix& A,
                               const rns8_matrix& B, const rns8_matrix& C) {
  if (!uses_rns_storage(plan.desc.semantics) || plan.prefix == 0) return RNS8_INVALID_ARGUMENT;
  if (A.backend != plan.backend || B.backend != plan.backend || C.backend != plan.backend)
    return RNS8_INVALID_ARGUMENT;
  if (A.device_id != ctx.device_id || B.device_id != ctx.device_id || C.device_id != ctx.device_id)
    return RNS8_INVALID_ARGUMENT;
  const uint32_t sp = storage_prefix(plan);
  const rns8_bound_kind bk = storage_bound_kind(plan);
  const uint32_t tm = plan.desc.tile_m, tn = plan.desc.tile_n;
  if (!matrix_matches(A, plan.desc.semantics, bk, plan.desc.m, plan.desc.k, sp, tm, tn) ||
      !matrix_matches(B, plan.desc.semantics, bk, plan.desc.k, plan.desc.n, sp, tm, tn) ||
      !matrix_matches(C, plan.desc.semantics, bk, plan.desc.m, plan.desc.n, sp, tm, tn))
    return RNS8_INVALID_ARGUMENT;
  if (!A.device_current || !B.device_current) return RNS8_INVALID_ARGUMENT;
  // C is written while A and B are read by other workgroups: no aliasing
  if (&A == &C || &B == &C) return RNS8_INVALID_ARGUMENT;
  return RNS8_SUCCESS;
}

// reference api_gemm.cpp:113-160
rns8_status check_finite_operands(const rns8_context& ctx, const rns8_plan& plan, uint16_t modulus,
                                  const rns8_matrix& A, const rns8_matrix& B, const rns8_matrix& C) {
  if (!uses_finite_storage(plan.desc.semantics) || !valid_finite_modulus(plan.desc.semantics, modulus) ||
      plan.desc.finite_modulus != modulus)
    return RNS8_INVALID_ARGUMENT;
  if (A.backend != plan.backend || B.backend != plan.backend || C.backend != plan.backend)
    return RNS8_INVALID_ARGUMENT;
  if (A.device_id != ctx.device_id || B.device_id != ctx.device_id || C.device_id != ctx.device_id)
    return RNS8_INVALID_ARGUMENT;
  if (!matrix_matches(A, plan.desc.semantics, RNS8_BOUND_NONE, plan.desc.m, plan.desc.k, 0) ||
      !matrix_matches(B, plan.desc.semantics, RNS8_BOUND_NONE, plan.desc.k, plan.desc.n, 0) ||
      !matrix_matches(C, plan.desc.semantics, RNS8_BOUND_NONE, plan.desc.m, plan.desc.n, 0))
    return RNS8_INVALID_ARGUMENT;
  if (!A.device_current || !B.device_current || A.finite_modulus != modulus || B.finite_modulus != modulus)
    return RNS8_INVALID_ARGUMENT;
  if (&A == &C || &B == &C) return RNS8_INVALID_ARGUMENT;
  return RNS8_SUCCESS;
}

// reference api_export.cpp:5-53
rns8_status check_export(const rns8_context& ctx, const rns8_plan& plan, const rns8_matrix& C,
                         rns8_semantics semantics) {
  if (plan.backend != ctx.backend || C.backend != plan.backend || plan.desc.semantics != semantics)
    return RNS8_INVALID_ARGUMENT;
  if (C.device_id != ctx.device_id || plan.device_id != ctx.device_id) return RNS8_INVALID_ARGUMENT;
  if (!matrix_matches(C, semantics, storage_bound_kind(plan), plan.desc.m, plan.desc.n, storage_prefix(plan),
                      plan.desc.tile_m, plan.desc.tile_n))
    return RNS8_INVALID_ARGUMENT;
  if (!C.device_current) return RNS8_INVALID_ARGUMENT;
  if (exact_wide(semantics) && C.exact_prefix != 0) {
    if (C.exact_prefix < plan.prefix) return RNS8_RANGE_ERROR;
    // a pending proof whose worst case fits needs no read back
    if (!exact_range_fits(semantics, C.exact_max, plan.product)) {
      if (!C.exact_pending) return RNS8_RANGE_ERROR;
      const rns8_status st = resolve_exact_proof(C, ctx.stream);
      if (st != RNS8_SUCCESS) return st;
      if (!exact_range_fits(semantics, C.exact_max, plan.product)) return RNS8_RANGE_ERROR;
    }
  }
  return RNS8_SUCCESS;
}

rns8_status check_finite_export(const rns8_context& ctx, const rns8_plan& plan, uint16_t modulus,
                                const rns8_matrix& C) {
  if (!uses_finite_storage(plan.desc.semantics) || plan.desc.finite_modulus != modulus ||
      !valid_finite_modulus(plan.desc.semantics, modulus))
    return RNS8_INVALID_ARGUMENT;
  if (plan.backend != ctx.backend || C.backend != plan.backend || C.device_id != ctx.device_id)
    return RNS8_INVALID_ARGUMENT;
  if (!matrix_matches(C, plan.desc.semantics, RNS8_BOUND_NONE, plan.desc.m, plan.desc.n, 0))
    return RNS8_INVALID_ARGUMENT;
  if (!C.device_current || C.finite_modulus != modulus) return RNS8_INVALID_ARGUMENT;
  return RNS8_SUCCESS;
}

// reference api_pack.cpp:31-76
rns8_status check_pack_native(const rns8_context& ctx, const rns8_matrix& m, int64_t ld, bool is_signed) {
  if (!valid_access(m.desc.rows, m.desc.cols, ld)) return RNS8_INVALID_ARGUMENT;
  const rns8_semantics bounded = is_signed ? RNS8_BOUNDED_I64 : RNS8_BOUNDED_U64;
  const rns8_semantics wide = is_signed ? RNS8_EXACT_WIDE_SIGNED : RNS8_EXACT_WIDE_UNSIGNED;
  if (m.desc.semantics != bounded && m.desc.semantics != wide) return RNS8_INVALID_ARGUMENT;
  if (ctx.backend != m.backend || m.device_id != ctx.device_id) return RNS8_INVALID_ARGUMENT;
  return RNS8_SUCCESS;
}

rns8_status check_pack_u8(const rns8_context& ctx, const rns8_matrix& m, uint16_t modulus, int64_t ld) {
  if (!valid_access(m.desc.rows, m.desc.cols, ld)) return RNS8_INVALID_ARGUMENT;
  if (!uses_finite_storage(m.desc.semantics) || !valid_finite_modulus(m.desc.semantics, modulus))
    return RNS8_INVALID_ARGUMENT;
  if (ctx.backend != m.backend || m.device_id != ctx.device_id) return RNS8_INVALID_ARGUMENT;
  return RNS8_SUCCESS;
}

GemmArgs gemm_args(const rns8_plan& plan, const rns8_matrix& A, const rns8_matrix& B, const rns8_matrix& C,
                   int8_t* splitk_ws, uint32_t nplanes, uint32_t slices) {
  GemmArgs g{};
  g.a = A.planes;
  g.b = B.planes;
  g.c = C.planes;
  g.m = plan.desc.m;
  g.n = plan.desc.n;
  g.k = plan.desc.k;
  g.lda = A.plane_ld;
  g.ldb = B.plane_ld;
  g.ldc = C.plane_ld;
  g.pitch_a = A.plane_pitch;
  g.pitch_b = B.plane_pitch;
  g.pitch_c = C.plane_pitch;
  g.nplanes = nplanes;
  g.slices = slices;
  g.splitk_ws = slices > 1 ? splitk_ws : nullptr;
  return g;
}

ExportArgs export_args(const rns8_plan& plan, const rns8_matrix& C, void* dst, int64_t ld, uint32_t limbs,
                       ExportKind kind, uint32_t* status) {
  return ExportArgs{C.planes, plan.desc.m, plan.desc.n, C.plane_ld, C.plane_pitch, dst, ld, limbs,
                    kind,     plan.desc.bound, status};
}

ExportU8Args export_u8_args(const rns8_plan& plan, const rns8_matrix& C, uint8_t* dst, int64_t ld, uint16_t modulus) {
  return ExportU8Args{C.planes, plan.desc.m, plan.desc.n, C.plane_ld, dst, ld, modulus};
}

PackArgs pack_args(const rns8_matrix& m, const void* src, int64_t ld, bool is_signed) {
  return PackArgs{src,      m.desc.rows, m.desc.cols, ld, m.planes, m.plane_ld, m.plane_pitch, m.prefix,
                  is_signed ? NativeKind::I64 : NativeKind::U64};
}

PackU8Args pack_u8_args(const rns8_matrix& m, const uint8_t* src, int64_t ld, uint16_t modulus) {
  return PackU8Args{src, m.desc.rows, m.desc.cols, ld, m.planes, m.plane_ld, modulus};
}

bool gemm_args_ok(const GemmArgs& a) {
  if (a.m <= 0 || a.n <= 0 || a.k <= 0) return false;
  if (a.nplanes == 0 || a.nplanes > kMaxPrefix) return false;
  if (a.lda % 16 || a.ldb % 16 || a.ldc % 16) return false;
  if (a.lda < a.k || a.ldb < a.n || a.ldc < a.n) return false;
  // 32-bit buffer offsets: a 256-row panel and a 64-row slab must stay below 2^31
  if (a.lda >= (int64_t{1} << 23) || a.ldb >= (int64_t{1} << 23)) return false;
  // unit decode runs in 32 bits: rows and tile origins below 2^31
  if (a.m >= (int64_t{1} << 31)) return false;
  if (a.ldc != a.ldb) return false;  // C columns == B columns: same padded pitch
  // (lda, ldb < 2^23 and m < 2^31 keep these products inside int64)
  if (a.pitch_a < a.m * a.lda || a.pitch_b < a.k * a.ldb || a.pitch_c < a.m * a.ldc) return false;
  if (!a.a || !a.b || !a.c) return false;
  if (a.slices == 0) return false;
  if (a.slices > 1 && !a.splitk_ws) return false;
  // the workspace holds [slices][planes][m][padded_ld(n)] residues
  if (a.slices > 1 && a.ldc != padded_ld(a.n)) return false;
  return true;
}

bool export_args_ok(const ExportArgs& a, uint32_t prefix) {
  if (!a.c || !a.dst || !a.status || a.m <= 0 || a.n <= 0 || a.ld < a.n) return false;
  if (prefix == 0 || prefix > kMaxPrefix) return false;
  if (a.ldc != padded_ld(a.n) || a.ldc / 4 > 0xFFFFFFFFll) return false;
  if (a.m > std::numeric_limits<int64_t>::max() / a.ldc || a.pitch_c < a.m * a.ldc || (a.pitch_c % 4) != 0)
    return false;
  if ((reinterpret_cast<uintptr_t>(a.c) & 3u) != 0) return false;
  if (a.limbs == 0 || a.limbs > 32) return false;
  if ((a.kind == ExportKind::I64 || a.kind == ExportKind::U64) && a.limbs != 1) return false;
  return true;
}

bool export_u8_args_ok(const ExportU8Args& a) {
  if (!a.c || !a.dst || a.m <= 0 || a.n <= 0 || a.ld < a.n) return false;
  if (a.ldc != padded_ld(a.n) || (reinterpret_cast<uintptr_t>(a.c) & 15u) != 0) return false;
  if (a.modulus < 2 || a.modulus > 256) return false;
  return a.ldc / 16 <= 0xFFFFFFFFll;
}

bool pack_args_ok(const PackArgs& a) {
  if (!a.src || !a.planes || a.rows <= 0 || a.cols <= 0 || a.ld < a.cols) return false;
  if (a.nplanes == 0 || a.nplanes > kMaxPrefix) return false;
  if (a.plane_ld != padded_ld(a.cols) || (a.plane_pitch % 16) != 0) return false;
  if (a.rows > std::numeric_limits<int64_t>::max() / a.plane_ld || a.plane_pitch < a.rows * a.plane_ld) return false;
  if ((reinterpret_cast<uintptr_t>(a.planes) & 15u) != 0) return false;
  // 8-column chunks numbered in 32 bits
  return (a.plane_ld / 8) * a.rows < (int64_t{1} << 32);
}

bool pack_u8_args_ok(const PackU8Args& a) {
  if (!a.src || !a.plane || a.rows <= 0 || a.cols <= 0 || a.ld < a.cols) return false;
  if (a.modulus < 2 || a.modulus > 256) return false;
  if (a.plane_ld != padded_ld(a.cols) || (reinterpret_cast<uintptr_t>(a.plane) & 15u) != 0) return false;
  // 16-column chunks numbered in 32 bits
  return a.rows <= (int64_t{1} << 32) / (a.plane_ld / 16) && (a.plane_ld / 16) * a.rows < (int64_t{1} << 32);
}

}  // namespace rns8x
