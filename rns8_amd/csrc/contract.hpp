// The host-side contract of pack -> GEMM -> export, with no device work:
// argument checks of the C ABI calls (statuses and their order follow the
// reference), the kernel arguments a validated call hands the launchers, and
// the launchers' own checks of those arguments. The ABI entry points and the
// launchers call these functions; tests/fuzz/fuzz_export_contract.cpp drives
// them with arbitrary descriptors and checks that every accepted call gives
// kernel arguments the launchers accept and whose reach stays inside the
// matrices' storage and the caller's buffers.
#pragma once

#include <cstdint>

#include "handles.hpp"
#include "kernels.hpp"

namespace rns8x {

// rows x cols elements at row stride ld (elements), and with `limbs` 64-bit
// limbs per element, addressable in int64 arithmetic.
bool valid_access(int64_t rows, int64_t cols, int64_t ld);
bool valid_limb_access(int64_t rows, int64_t cols, int64_t ld, uint32_t limbs);

// rns8_create_matrix's validation and storage layout (planes, pitches,
// bytes); the caller then allocates plane_bytes of planes.
rns8_status init_matrix(const rns8_matrix_desc& d, rns8_backend_kind backend, int device_id, rns8_matrix& m);

// reference api_gemm.cpp:50-160, api_export.cpp:5-53, api_pack.cpp:31-76
rns8_status check_plan_ctx_ws(const rns8_context& ctx, const rns8_plan& plan, const rns8_workspace& ws);
rns8_status check_rns_operands(const rns8_context& ctx, const rns8_plan& plan, const rns8_matrix& A,
                               const rns8_matrix& B, const rns8_matrix& C);
rns8_status check_finite_operands(const rns8_context& ctx, const rns8_plan& plan, uint16_t modulus,
                                  const rns8_matrix& A, const rns8_matrix& B, const rns8_matrix& C);
rns8_status check_export(const rns8_context& ctx, const rns8_plan& plan, const rns8_matrix& C,
                         rns8_semantics semantics);
rns8_status check_finite_export(const rns8_context& ctx, const rns8_plan& plan, uint16_t modulus,
                                const rns8_matrix& C);
// pack of 64-bit elements (is_signed: int64) into a bounded or exact-wide matrix
rns8_status check_pack_native(const rns8_context& ctx, const rns8_matrix& m, int64_t ld, bool is_signed);
rns8_status check_pack_u8(const rns8_context& ctx, const rns8_matrix& m, uint16_t modulus, int64_t ld);

// Kernel arguments of a validated call (the planes of A, B and C as stored).
GemmArgs gemm_args(const rns8_plan& plan, const rns8_matrix& A, const rns8_matrix& B, const rns8_matrix& C,
                   int8_t* splitk_ws, uint32_t nplanes, uint32_t slices);
ExportArgs export_args(const rns8_plan& plan, const rns8_matrix& C, void* dst, int64_t ld, uint32_t limbs,
                       ExportKind kind, uint32_t* status);
ExportU8Args export_u8_args(const rns8_plan& plan, const rns8_matrix& C, uint8_t* dst, int64_t ld, uint16_t modulus);
PackArgs pack_args(const rns8_matrix& m, const void* src, int64_t ld, bool is_signed);
PackU8Args pack_u8_args(const rns8_matrix& m, const uint8_t* src, int64_t ld, uint16_t modulus);

// The launchers' own checks of these arguments (gemm_args_ok,
// export_args_ok, export_u8_args_ok, pack_args_ok, pack_u8_args_ok) are
// declared in kernels.hpp beside the launchers and defined in contract.cpp.

}  // namespace rns8x
