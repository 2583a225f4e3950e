// Handle state behind the opaque rns8 ABI types, plus shared host helpers.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "rns8/rns8.h"
#include "rns8_mi355x.h"
#include "host_copy.hpp"
#include "kernels.hpp"
#include "tables.hpp"
#include "exact_axes.hpp"
#include "exact_range.hpp"
#include "wide_int.hpp"


namespace rns8x {
struct OneshotCache;
}

struct rns8_context {
  rns8_backend_kind backend = RNS8_BACKEND_HIP_DIRECT;
  int device_id = 0;
  hipStream_t stream = nullptr;
  rns8_device_info device_info{};
  rns8x::HostStaging host;  // pinned staging for host-memory operands and results
  // device state (plan, matrices, workspace) of the last oneshot call, reused
  // by the next oneshot call with an equal descriptor; freed with the context
  rns8x::OneshotCache* oneshot = nullptr;
};

// Per-tile bounded schedule (reference src/core/internal.hpp:22-70, the
// rns8_plan schedule_* fields and tile_schedule). For a per-tile plan `entries`
// lists every tile's prefixes; it is empty when every tile runs the plan
// prefix without flags (the schedule collapses), and always empty for global
// plans.
struct TileSchedule {
  std::vector<uint64_t> bounds;
  std::vector<rns8_plan_tile_schedule_entry> entries;
  std::vector<uint8_t> zero_a_rows, zero_b_cols;
  uint32_t min_required = 0, max_required = 0, min_selected = 0, max_selected = 0;
  uint32_t groups = 0, adaptive_prefix = 0, adaptive_skip = 0, range_bits = 0, flags = 0;
  uint64_t zero_a_row_count = 0, zero_b_col_count = 0, zero_row_col_product_count = 0;
};

struct rns8_plan {
  rns8_gemm_desc desc{};  // caller descriptor; max_prefix holds the budget, tiles defaulted to 128
  rns8_backend_kind backend = RNS8_BACKEND_HIP_DIRECT;
  int device_id = 0;
  uint32_t budget = 0;           // max_prefix after defaulting
  uint32_t prefix = 0;           // selected prefix (0 for finite semantics)
  uint32_t required_prefix = 0;  // minimum proven prefix
  uint32_t range_bits = 0;       // bit length of the required CRT range
  rns8x::I256 product;           // modulus product of the selected prefix
  uint64_t tile_rows = 0, tile_cols = 0, tile_count = 0;
  uint32_t splitk_slices = 1;
  uint64_t splitk_bytes = 0;  // workspace bytes: the larger of the split-K and the fused path's needs
  // Bounded int64/uint64 plans whose output is small enough for the fused
  // native-input GEMM (fused.hip): its K split and partial-residue bytes.
  bool fused_ok = false;
  rns8x::FusedShape fused{};
  TileSchedule schedule;  // per-tile bound kinds only
  // Per-tile plans: device lists the GEMM and export run from, built when the
  // plan is created and never changed. `units` (two words per unit, see
  // launch_gemm_listed) is empty when every tile runs the plan prefix; then
  // the ordinary GEMM runs. `export_tiles` holds one record per tile, ordered
  // by selected prefix, in `export_groups`; prefix 0 marks zero-output tiles.
  struct ExportGroup {
    uint32_t prefix, first, count;
  };
  uint32_t* units = nullptr;
  uint32_t unit_count = 0;
  uint32_t unit_edge = 0;  // 256 or 128: output tile edge of a listed unit
  rns8x::TileFill* zero_fills = nullptr;
  uint32_t zero_fill_count = 0;
  rns8x::TileExport* export_tiles = nullptr;
  std::vector<ExportGroup> export_groups;
};

struct rns8_matrix {
  rns8_matrix_desc desc{};
  rns8_backend_kind backend = RNS8_BACKEND_HIP_DIRECT;
  int device_id = 0;
  uint64_t instance_id = 0;
  uint32_t prefix = 0;  // residue planes held (1 for finite storage)
  uint16_t finite_modulus = 0;
  uint64_t source_version = 0;
  bool device_current = false;
  // planes in HBM, layout rns8_mi355x_planes_v1 (tables.hpp)
  int8_t* planes = nullptr;
  int64_t plane_ld = 0;
  int64_t plane_pitch = 0;
  uint64_t plane_bytes = 0;
  // exact-wide proofs (reference exact_range.hpp): exact_prefix == 0 means
  // no proof. The proof lies on the device, in one of two sets of
  // proof_device (layout below): per-row and per-column axis records and 8
  // words, the proof's bound in words 0..3. proof_kind says what set
  // proof_set holds: native axes (a pack), carried axes (a GEMM result whose
  // summaries were computed), or a lazy proof: the snapshot of a GEMM's
  // operand axes (A's rows of kind lazy_rows, B's columns of kind lazy_cols,
  // maxA in words 0..3, maxB in 4..7, inner dimension lazy_k), from which
  // the result's own summaries are computed when a decision needs them. The
  // other set is free: writers fill it and then make it current, so a
  // refused call leaves the current proof as it was. exact_max is a bound
  // the proof's bound never exceeds, exact unless exact_pending: a decision
  // that it passes is the exact decision, and the device bound is read back
  // (after proof_event, recorded by the last proof writer) when one needs it.
  // Proof work is ordered on streams like the planes it describes.
  enum class ProofKind : uint8_t { Native, Carried, Uniform, Lazy };
  mutable rns8x::I512 exact_max;
  uint32_t exact_prefix = 0;
  mutable bool exact_pending = false;
  mutable ProofKind proof_kind = ProofKind::Native;
  mutable uint32_t proof_set = 0;
  uint32_t lazy_rows = 0, lazy_cols = 0;  // rns8x::xa::AxisKind of a lazy proof's snapshot
  uint64_t lazy_k = 0;
  // [words set 0 (8)] [words set 1 (8)] [set 0 rows] [set 0 cols] [set 1
  // rows] [set 1 cols] [pack scratch: the per-tile partials of the rows,
  // then of the columns (rns8x::native_partial_rows / _cols)]
  uint8_t* proof_device = nullptr;
  hipEvent_t proof_event = nullptr;
  static uint64_t proof_bytes(int64_t rows, int64_t cols) {
    return 128u + 2u * static_cast<uint64_t>(rows + cols) * sizeof(rns8x::xa::AxisRecord) +
           static_cast<uint64_t>(rns8x::native_partial_rows(rows, cols) + rns8x::native_partial_cols(rows, cols)) *
               sizeof(rns8x::xa::AxisPartial);
  }
  uint64_t* proof_words(uint32_t set) const { return reinterpret_cast<uint64_t*>(proof_device) + 8u * set; }
  rns8x::xa::AxisRecord* proof_rows(uint32_t set) const {
    return reinterpret_cast<rns8x::xa::AxisRecord*>(proof_device + 128) + (desc.rows + desc.cols) * set;
  }
  rns8x::xa::AxisRecord* proof_cols(uint32_t set) const { return proof_rows(set) + desc.rows; }
  rns8x::xa::AxisPartial* row_partials() const {
    return reinterpret_cast<rns8x::xa::AxisPartial*>(proof_rows(2));
  }
  rns8x::xa::AxisPartial* col_partials() const {
    return row_partials() + rns8x::native_partial_rows(desc.rows, desc.cols);
  }
  // cached staging buffers (export is logically const, reference
  // api_export.cpp:276-287 keeps the same kind of cache on the matrix)
  void* upload = nullptr;
  std::size_t upload_bytes = 0;
  void* staging = nullptr;
  std::size_t staging_bytes = 0;
  uint32_t* status = nullptr;
};

struct rns8_workspace {
  rns8_backend_kind backend = RNS8_BACKEND_HIP_DIRECT;
  rns8_semantics semantics = RNS8_BOUNDED_I64;
  rns8_bound_kind bound_kind = RNS8_BOUND_NONE;
  int64_t m = 0, n = 0, k = 0;
  uint32_t prefix = 0;
  uint32_t finite_modulus = 0;
  int device_id = 0;
  int8_t* splitk = nullptr;
  uint64_t splitk_bytes = 0;
};

// Handles for entry points this library does not execute; never created.
struct rns8_sparse_matrix {
  int unused;
};
struct rns8_prepack_cache {
  int unused;
};
struct rns8_result_cache {
  int unused;
};

namespace rns8x {

template <typename F>
rns8_status guard(F&& f) {
  try {
    return f();
  } catch (...) {
    return RNS8_INTERNAL_ERROR;
  }
}

inline bool valid_abi(uint64_t struct_size, uint32_t abi_version, std::size_t expected) {
  return abi_version == RNS8_ABI_VERSION && struct_size >= expected;
}

void copy_text(char* dst, std::size_t size, const char* src);

// out-struct helper: keep caller's size/version, zero the rest
template <typename T>
void reset_out(T& out) {
  const uint64_t size = out.struct_size;
  const uint32_t version = out.abi_version;
  out = T{};
  out.struct_size = size;
  out.abi_version = version;
}

bool uses_rns_storage(rns8_semantics s);
bool uses_finite_storage(rns8_semantics s);
bool exact_wide(rns8_semantics s);
uint32_t default_prefix(rns8_semantics s);
I256 modulus_product(uint32_t prefix);
uint32_t required_prefix_for_range(const I256& range);
bool valid_finite_modulus(rns8_semantics s, uint32_t modulus);

// reference moduli.cpp:295-387 (validate_gemm_desc)
rns8_status validate_gemm_desc(const rns8_gemm_desc& d, uint32_t prefix);
// reference moduli.cpp:389-448 (validate_matrix_desc)
rns8_status validate_matrix_desc(const rns8_matrix_desc& d, uint32_t prefix);
// reference moduli.cpp:234-293 (validate_bound_contract)
rns8_status validate_bound_contract(rns8_semantics s, rns8_bound_kind bk, uint64_t bound, uint32_t prefix);
// validation + prefix selection shared by plan creation and select_prefix
rns8_status plan_prefix(const rns8_gemm_desc& d, uint32_t& budget, uint32_t& selected, uint32_t& required,
                        uint32_t& range_bits, uint64_t& effective_bound);

// Frees the context's cached oneshot state (api_exec.cpp).
void release_oneshot_cache(rns8_context& ctx);

// HIP helpers
rns8_status hip_status(hipError_t e);
rns8_status ensure_device_buffer(int device, void** ptr, std::size_t* have, std::size_t need);
void free_device(void* p);
hipStream_t pick_stream(const rns8_context& ctx, void* stream);

// matrix storage: storage prefix / bound kind a plan expects of its operands
uint32_t storage_prefix(const rns8_plan& p);
bool per_tile_kind(rns8_bound_kind b);
// plan state that needs no device (validation, prefixes, tiles, schedule)
rns8_status init_plan(const rns8_gemm_desc& d, rns8_backend_kind backend, rns8_plan& plan);
// reference api_plan_schedule.inc:109-261 (per-tile branch)
rns8_status build_tile_schedule(const rns8_gemm_desc& d, uint32_t budget, TileSchedule& s);
// rns8_get_plan_tile_schedule's entries for a plan (api_plan_public_api.inc:119-160)
void plan_tile_entries(const rns8_plan& p, rns8_plan_tile_schedule_entry* out);
// Builds and uploads a per-tile plan's device lists (no-op for other plans);
// the current device must be the plan's.
rns8_status upload_tile_lists(rns8_plan& p, hipStream_t stream);
void free_tile_lists(rns8_plan& p);
rns8_bound_kind storage_bound_kind(const rns8_plan& p);
bool matrix_matches(const rns8_matrix& m, rns8_semantics s, rns8_bound_kind bk, int64_t rows, int64_t cols,
                    uint32_t prefix, uint32_t tile_m = 0, uint32_t tile_n = 0);

}  // namespace rns8x
