// rns8 ABI: contracts, prefix selection, context/plan/matrix/workspace
// lifetime and introspection (HIP_DIRECT on gfx950).
//
// Validation and status precedence restate the reference's rules so callers
// see the same status for the same descriptor:
//   src/core/moduli.cpp:164-448        ladder products, prefix, descriptor checks
//   src/core/api_plan_public_api.inc   plan creation order of checks
//   src/core/api_plan_schedule.inc     global-bound prefix schedule
//   src/core/api_matrix_public_api.inc matrix creation
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>
#include <new>

#include "contract.hpp"
#include "handles.hpp"
#include "kernels.hpp"

namespace rns8x {

// no allocation: the getters that call it leave their outputs whole
void copy_text(char* dst, std::size_t size, const char* src) {
  if (size == 0) return;
  const std::size_t n = src ? strnlen(src, size - 1) : 0;
  if (n) std::memcpy(dst, src, n);
  dst[n] = '\0';
}

bool uses_rns_storage(rns8_semantics s) {
  return s == RNS8_BOUNDED_I64 || s == RNS8_BOUNDED_U64 || s == RNS8_EXACT_WIDE_SIGNED ||
         s == RNS8_EXACT_WIDE_UNSIGNED;
}
bool uses_finite_storage(rns8_semantics s) { return s == RNS8_FINITE_RING_U8 || s == RNS8_FINITE_FIELD_U8; }
bool exact_wide(rns8_semantics s) { return s == RNS8_EXACT_WIDE_SIGNED || s == RNS8_EXACT_WIDE_UNSIGNED; }

static bool known_semantics(rns8_semantics s) {
  switch (s) {
    case RNS8_BOUNDED_I64:
    case RNS8_BOUNDED_U64:
    case RNS8_EXACT_WIDE_SIGNED:
    case RNS8_EXACT_WIDE_UNSIGNED:
    case RNS8_WRAP_U64_MOD_2_64:
    case RNS8_FINITE_RING_U8:
    case RNS8_FINITE_FIELD_U8:
      return true;
    default:
      return false;
  }
}
static bool known_bound_kind(rns8_bound_kind b) {
  return static_cast<uint32_t>(b) <= static_cast<uint32_t>(RNS8_BOUND_INPUT_RANGE_AND_K);
}
static bool known_layout(rns8_layout l) { return l == RNS8_LAYOUT_ROW_MAJOR || l == RNS8_LAYOUT_COLUMN_MAJOR; }
static bool per_tile(rns8_bound_kind b) {
  return b == RNS8_BOUND_PER_TILE_MAX_ABS || b == RNS8_BOUND_PER_TILE_MAX_UNSIGNED;
}
static bool valid_tile_size(uint32_t v) { return v == 0 || (v >= 64 && v <= 512 && (v & (v - 1u)) == 0); }
static bool valid_zero_mask(const uint8_t* mask, uint64_t count, int64_t expected) {
  if (!mask || expected < 0 || count != static_cast<uint64_t>(expected)) return false;
  for (uint64_t i = 0; i < count; ++i)
    if (mask[i] > 1u) return false;
  return true;
}

uint32_t default_prefix(rns8_semantics s) {
  switch (s) {
    case RNS8_BOUNDED_I64:
    case RNS8_BOUNDED_U64:
      return RNS8_DEFAULT_BOUNDED_PREFIX;
    case RNS8_EXACT_WIDE_SIGNED:
    case RNS8_EXACT_WIDE_UNSIGNED:
      return RNS8_MAX_SUPPORTED_PREFIX;
    default:
      return 0;
  }
}

I256 modulus_product(uint32_t prefix) {
  I256 p = I256::from_u64(1);
  for (uint32_t i = 0; i < prefix && i < kLadderSize; ++i) p = p * I256::from_u64(kLadder[i]);
  return p;
}

uint32_t required_prefix_for_range(const I256& range) {
  I256 p = I256::from_u64(1);
  for (uint32_t prefix = 1; prefix <= kMaxPrefix; ++prefix) {
    p = p * I256::from_u64(kLadder[prefix - 1]);
    if (p > range) return prefix;
  }
  return 0;
}

bool valid_finite_modulus(rns8_semantics s, uint32_t modulus) {
  if (s == RNS8_FINITE_RING_U8) return modulus >= 2 && modulus <= 256;
  if (s == RNS8_FINITE_FIELD_U8) {
    if (modulus < 2 || modulus > 251) return false;
    for (uint32_t d = 2; d * d <= modulus; ++d)
      if (modulus % d == 0) return false;
    return true;
  }
  return false;
}

// reference moduli.cpp:208-232
static bool input_range_output_bound(const rns8_gemm_desc& d, uint64_t& out) {
  out = 0;
  if (d.bound_kind != RNS8_BOUND_INPUT_RANGE_AND_K ||
      (d.semantics != RNS8_BOUNDED_I64 && d.semantics != RNS8_BOUNDED_U64) || d.k <= 0)
    return false;
  if (d.semantics == RNS8_BOUNDED_I64 && (d.lhs_bound > (uint64_t{1} << 63) || d.rhs_bound > (uint64_t{1} << 63)))
    return false;
  const I256 product =
      I256::from_u64(static_cast<uint64_t>(d.k)) * I256::from_u64(d.lhs_bound) * I256::from_u64(d.rhs_bound);
  const I256 limit = d.semantics == RNS8_BOUNDED_I64 ? I256::pow2(63) : I256::from_u64(UINT64_MAX);
  if (product > limit) return false;
  out = product.w[0];
  return true;
}

rns8_status validate_bound_contract(rns8_semantics s, rns8_bound_kind bk, uint64_t bound, uint32_t prefix) {
  if (!known_semantics(s) || !known_bound_kind(bk)) return RNS8_INVALID_ARGUMENT;
  if (prefix == 0 || prefix > kMaxPrefix) return RNS8_INVALID_ARGUMENT;
  const I256 product = modulus_product(prefix);
  switch (s) {
    case RNS8_BOUNDED_I64: {
      if (bk == RNS8_BOUND_INPUT_RANGE_AND_K) return RNS8_UNSUPPORTED_BACKEND;
      if (bk == RNS8_BOUND_PER_TILE_MAX_ABS) return bound == 0 ? RNS8_SUCCESS : RNS8_INVALID_ARGUMENT;
      if (bk == RNS8_BOUND_NONE || bk == RNS8_BOUND_GLOBAL_MAX_UNSIGNED || bk == RNS8_BOUND_PER_TILE_MAX_UNSIGNED)
        return RNS8_INVALID_ARGUMENT;
      if (bk != RNS8_BOUND_GLOBAL_MAX_ABS) return RNS8_UNSUPPORTED_BACKEND;
      if (bound > (uint64_t{1} << 63)) return RNS8_INVALID_ARGUMENT;
      return product > I256::from_u64(bound) * I256::from_u64(2) ? RNS8_SUCCESS : RNS8_RANGE_ERROR;
    }
    case RNS8_BOUNDED_U64: {
      if (bk == RNS8_BOUND_INPUT_RANGE_AND_K) return RNS8_UNSUPPORTED_BACKEND;
      if (bk == RNS8_BOUND_PER_TILE_MAX_UNSIGNED) return bound == 0 ? RNS8_SUCCESS : RNS8_INVALID_ARGUMENT;
      if (bk == RNS8_BOUND_NONE || bk == RNS8_BOUND_GLOBAL_MAX_ABS || bk == RNS8_BOUND_PER_TILE_MAX_ABS)
        return RNS8_INVALID_ARGUMENT;
      if (bk != RNS8_BOUND_GLOBAL_MAX_UNSIGNED) return RNS8_UNSUPPORTED_BACKEND;
      return product > I256::from_u64(bound) ? RNS8_SUCCESS : RNS8_RANGE_ERROR;
    }
    default:
      return RNS8_UNSUPPORTED_BACKEND;
  }
}

rns8_status validate_gemm_desc(const rns8_gemm_desc& d, uint32_t prefix) {
  if (!valid_abi(d.struct_size, d.abi_version, sizeof(d))) return RNS8_INVALID_ARGUMENT;
  if (d.m <= 0 || d.n <= 0 || d.k <= 0) return RNS8_INVALID_ARGUMENT;
  constexpr uint32_t allowed =
      RNS8_PLAN_FORCE_FIXED_PREFIX | RNS8_PLAN_ALLOW_PROVEN_ZERO_TILE_SKIPS | RNS8_PLAN_ALLOW_PROVEN_ZERO_ROW_COL_SKIPS;
  if ((d.flags & ~allowed) != 0) return RNS8_INVALID_ARGUMENT;
  const bool fixed = (d.flags & RNS8_PLAN_FORCE_FIXED_PREFIX) != 0;
  const bool zero_tiles = (d.flags & RNS8_PLAN_ALLOW_PROVEN_ZERO_TILE_SKIPS) != 0;
  const bool zero_rowcol = (d.flags & RNS8_PLAN_ALLOW_PROVEN_ZERO_ROW_COL_SKIPS) != 0;
  if (!valid_tile_size(d.tile_m) || !valid_tile_size(d.tile_n)) return RNS8_INVALID_ARGUMENT;
  const bool tiles = per_tile(d.bound_kind);
  if (!tiles && (d.tile_bounds || d.tile_bounds_count != 0)) return RNS8_INVALID_ARGUMENT;
  if (!zero_rowcol && (d.zero_a_rows || d.zero_a_rows_count != 0 || d.zero_b_cols || d.zero_b_cols_count != 0))
    return RNS8_INVALID_ARGUMENT;
  if (zero_tiles && !tiles) return RNS8_INVALID_ARGUMENT;
  if (zero_rowcol && (!tiles || !valid_zero_mask(d.zero_a_rows, d.zero_a_rows_count, d.m) ||
                      !valid_zero_mask(d.zero_b_cols, d.zero_b_cols_count, d.n)))
    return RNS8_INVALID_ARGUMENT;
  if (!known_semantics(d.semantics) || !known_bound_kind(d.bound_kind)) return RNS8_INVALID_ARGUMENT;
  if (!uses_finite_storage(d.semantics) && d.finite_modulus != 0) return RNS8_INVALID_ARGUMENT;
  if (d.bound_kind != RNS8_BOUND_INPUT_RANGE_AND_K && (d.lhs_bound != 0 || d.rhs_bound != 0))
    return RNS8_INVALID_ARGUMENT;
  if (exact_wide(d.semantics)) {
    if (d.bound_kind != RNS8_BOUND_NONE || d.bound != 0) return RNS8_INVALID_ARGUMENT;
    if (prefix == 0 || prefix > kMaxPrefix) return RNS8_INVALID_ARGUMENT;
    const I256 required = I256::from_u64(static_cast<uint64_t>(d.k)) *
                          I256::pow2(d.semantics == RNS8_EXACT_WIDE_SIGNED ? 127u : 128u);
    return modulus_product(prefix) > required ? RNS8_SUCCESS : RNS8_RANGE_ERROR;
  }
  if (d.semantics == RNS8_WRAP_U64_MOD_2_64) {
    if (d.bound_kind != RNS8_BOUND_NONE || d.bound != 0 || prefix != 0 || fixed) return RNS8_INVALID_ARGUMENT;
    return RNS8_SUCCESS;
  }
  if (uses_finite_storage(d.semantics)) {
    if (d.bound_kind != RNS8_BOUND_NONE || d.bound != 0 || d.max_prefix != 0 || prefix != 0 || fixed ||
        !valid_finite_modulus(d.semantics, d.finite_modulus))
      return RNS8_INVALID_ARGUMENT;
    return RNS8_SUCCESS;
  }
  if (d.bound_kind == RNS8_BOUND_INPUT_RANGE_AND_K) {
    if (d.bound != 0 || d.tile_bounds || d.tile_bounds_count != 0) return RNS8_INVALID_ARGUMENT;
    uint64_t out = 0;
    if (!input_range_output_bound(d, out)) return RNS8_RANGE_ERROR;
    if (prefix == 0 || prefix > kMaxPrefix) return RNS8_INVALID_ARGUMENT;
    const I256 required = d.semantics == RNS8_BOUNDED_I64 ? I256::from_u64(out) * I256::from_u64(2)
                                                          : I256::from_u64(out);
    return modulus_product(prefix) > required ? RNS8_SUCCESS : RNS8_RANGE_ERROR;
  }
  return validate_bound_contract(d.semantics, d.bound_kind, d.bound, prefix);
}

rns8_status validate_matrix_desc(const rns8_matrix_desc& d, uint32_t prefix) {
  if (!valid_abi(d.struct_size, d.abi_version, sizeof(d))) return RNS8_INVALID_ARGUMENT;
  if (d.rows <= 0 || d.cols <= 0 || d.flags != 0) return RNS8_INVALID_ARGUMENT;
  if (!known_semantics(d.semantics) || !known_bound_kind(d.bound_kind) || !known_layout(d.logical_layout))
    return RNS8_INVALID_ARGUMENT;
  if (d.logical_ld != 0 && d.logical_ld < d.cols) return RNS8_INVALID_ARGUMENT;
  if (!valid_tile_size(d.tile_m) || !valid_tile_size(d.tile_n)) return RNS8_INVALID_ARGUMENT;
  const bool column_major = d.logical_layout == RNS8_LAYOUT_COLUMN_MAJOR;
  switch (d.semantics) {
    case RNS8_BOUNDED_I64:
      if (prefix == 0 || prefix > kMaxPrefix) return RNS8_INVALID_ARGUMENT;
      if (d.bound_kind != RNS8_BOUND_GLOBAL_MAX_ABS && d.bound_kind != RNS8_BOUND_PER_TILE_MAX_ABS)
        return RNS8_INVALID_ARGUMENT;
      return column_major ? RNS8_UNSUPPORTED_BACKEND : RNS8_SUCCESS;
    case RNS8_BOUNDED_U64:
      if (prefix == 0 || prefix > kMaxPrefix) return RNS8_INVALID_ARGUMENT;
      if (d.bound_kind != RNS8_BOUND_GLOBAL_MAX_UNSIGNED && d.bound_kind != RNS8_BOUND_PER_TILE_MAX_UNSIGNED)
        return RNS8_INVALID_ARGUMENT;
      return column_major ? RNS8_UNSUPPORTED_BACKEND : RNS8_SUCCESS;
    case RNS8_EXACT_WIDE_SIGNED:
    case RNS8_EXACT_WIDE_UNSIGNED:
      if (prefix == 0 || prefix > kMaxPrefix) return RNS8_INVALID_ARGUMENT;
      if (d.bound_kind != RNS8_BOUND_NONE) return RNS8_INVALID_ARGUMENT;
      return column_major ? RNS8_UNSUPPORTED_BACKEND : RNS8_SUCCESS;
    case RNS8_WRAP_U64_MOD_2_64:
      if (d.bound_kind != RNS8_BOUND_NONE || prefix != 0) return RNS8_INVALID_ARGUMENT;
      return column_major ? RNS8_UNSUPPORTED_BACKEND : RNS8_SUCCESS;
    case RNS8_FINITE_RING_U8:
    case RNS8_FINITE_FIELD_U8:
      if (prefix != 0 || d.max_prefix != 0 || d.bound_kind != RNS8_BOUND_NONE) return RNS8_INVALID_ARGUMENT;
      return column_major ? RNS8_UNSUPPORTED_BACKEND : RNS8_SUCCESS;
    default:
      return RNS8_INVALID_ARGUMENT;
  }
}

// Validation + global prefix schedule (reference api_plan_public_api.inc:3-60
// and api_plan_schedule.inc:109-279 global branch). Backend routing is left
// to the caller.
rns8_status plan_prefix(const rns8_gemm_desc& d, uint32_t& budget, uint32_t& selected, uint32_t& required,
                        uint32_t& range_bits, uint64_t& effective_bound) {
  if (!valid_abi(d.struct_size, d.abi_version, sizeof(d))) return RNS8_INVALID_ARGUMENT;
  budget = d.max_prefix == 0 ? default_prefix(d.semantics) : d.max_prefix;
  const rns8_status v = validate_gemm_desc(d, budget);
  if (v != RNS8_SUCCESS) return v;
  // the schedule's tile grid must have a representable tile count, for every
  // plan (reference api_plan_schedule.inc:113-118)
  {
    const uint64_t tm = d.tile_m == 0 ? 128u : d.tile_m, tn = d.tile_n == 0 ? 128u : d.tile_n;
    const uint64_t rows = (static_cast<uint64_t>(d.m) + tm - 1) / tm;
    const uint64_t cols = (static_cast<uint64_t>(d.n) + tn - 1) / tn;
    if (cols != 0 && rows > std::numeric_limits<uint64_t>::max() / cols) return RNS8_RANGE_ERROR;
  }
  effective_bound = d.bound;
  if (d.bound_kind == RNS8_BOUND_INPUT_RANGE_AND_K && !input_range_output_bound(d, effective_bound))
    return RNS8_RANGE_ERROR;
  selected = 0;
  required = 0;
  range_bits = 0;
  if (uses_finite_storage(d.semantics) || d.semantics == RNS8_WRAP_U64_MOD_2_64) return RNS8_SUCCESS;
  I256 range;
  switch (d.semantics) {
    case RNS8_BOUNDED_I64:
      range = I256::from_u64(effective_bound) * I256::from_u64(2);
      break;
    case RNS8_BOUNDED_U64:
      range = I256::from_u64(effective_bound);
      break;
    case RNS8_EXACT_WIDE_SIGNED:
      range = I256::from_u64(static_cast<uint64_t>(d.k)) * I256::pow2(127);
      break;
    default:
      range = I256::from_u64(static_cast<uint64_t>(d.k)) * I256::pow2(128);
      break;
  }
  range_bits = range.bit_length();
  if (per_tile(d.bound_kind)) {
    // the plan prefix is the budget; each tile selects its own (build_tile_schedule)
    TileSchedule sched;
    const rns8_status st = build_tile_schedule(d, budget, sched);
    if (st != RNS8_SUCCESS) return st;
    selected = budget;
    required = sched.min_required;
    range_bits = sched.range_bits;
    return RNS8_SUCCESS;
  }
  required = required_prefix_for_range(range);
  if (required == 0 || required > budget) return RNS8_RANGE_ERROR;
  selected = (d.flags & RNS8_PLAN_FORCE_FIXED_PREFIX) ? budget : required;
  return RNS8_SUCCESS;
}

rns8_status hip_status(hipError_t e) { return e == hipSuccess ? RNS8_SUCCESS : RNS8_BACKEND_FAILURE; }

rns8_status ensure_device_buffer(int device, void** ptr, std::size_t* have, std::size_t need) {
  if (*ptr && *have >= need) return RNS8_SUCCESS;
  if (hipSetDevice(device) != hipSuccess) return RNS8_BACKEND_FAILURE;
  if (*ptr) {
    (void)hipFree(*ptr);
    *ptr = nullptr;
    *have = 0;
  }
  void* p = nullptr;
  if (hipMalloc(&p, need ? need : 16) != hipSuccess) return RNS8_BACKEND_FAILURE;
  *ptr = p;
  *have = need;
  return RNS8_SUCCESS;
}

void free_device(void* p) {
  if (p) (void)hipFree(p);
}

hipStream_t pick_stream(const rns8_context& ctx, void* stream) {
  return stream ? static_cast<hipStream_t>(stream) : ctx.stream;
}

bool per_tile_kind(rns8_bound_kind b) { return per_tile(b); }

// reference api_plan_schedule.inc:46-52: a per-tile plan stores only the
// planes its tiles select
uint32_t storage_prefix(const rns8_plan& p) {
  if (uses_finite_storage(p.desc.semantics)) return 0u;
  if (per_tile(p.desc.bound_kind) && p.schedule.max_selected > 0) return p.schedule.max_selected;
  return p.prefix;
}

namespace {

// reference api_plan_schedule.inc:54-72 (make_tile_schedule_entry)
rns8_plan_tile_schedule_entry tile_entry(int64_t m, int64_t n, uint32_t tile_m, uint32_t tile_n, uint64_t tile_cols,
                                         uint64_t index, uint32_t required, uint32_t selected, uint32_t range_bits,
                                         uint32_t flags) {
  rns8_plan_tile_schedule_entry e{};
  e.struct_size = sizeof(e);
  e.abi_version = RNS8_ABI_VERSION;
  e.flags = flags;
  e.tile_row = index / tile_cols;
  e.tile_col = index % tile_cols;
  e.row_offset = static_cast<int64_t>(e.tile_row * tile_m);
  e.col_offset = static_cast<int64_t>(e.tile_col * tile_n);
  e.row_extent = std::min<int64_t>(tile_m, m - e.row_offset);
  e.col_extent = std::min<int64_t>(tile_n, n - e.col_offset);
  e.required_prefix = required;
  e.selected_prefix = selected;
  e.range_bit_length = range_bits;
  return e;
}

// reference api_plan_schedule.inc:35-38
I256 tile_range(rns8_semantics s, uint64_t bound) {
  return s == RNS8_BOUNDED_I64 ? I256::from_u64(bound) * I256::from_u64(2) : I256::from_u64(bound);
}

}  // namespace

rns8_status build_tile_schedule(const rns8_gemm_desc& d, uint32_t budget, TileSchedule& s) {
  s = TileSchedule{};
  const uint32_t tm = d.tile_m == 0 ? 128u : d.tile_m;
  const uint32_t tn = d.tile_n == 0 ? 128u : d.tile_n;
  const uint64_t rows = (static_cast<uint64_t>(d.m) + tm - 1) / tm;
  const uint64_t cols = (static_cast<uint64_t>(d.n) + tn - 1) / tn;
  const uint64_t count = rows * cols;
  const bool proofs = (d.flags & RNS8_PLAN_ALLOW_PROVEN_ZERO_ROW_COL_SKIPS) != 0;
  if (cols != 0 && rows > std::numeric_limits<uint64_t>::max() / cols) return RNS8_RANGE_ERROR;
  if (proofs) {
    s.zero_a_rows.assign(d.zero_a_rows, d.zero_a_rows + d.zero_a_rows_count);
    s.zero_b_cols.assign(d.zero_b_cols, d.zero_b_cols + d.zero_b_cols_count);
    for (uint8_t v : s.zero_a_rows) s.zero_a_row_count += v != 0;
    for (uint8_t v : s.zero_b_cols) s.zero_b_col_count += v != 0;
    // the count of proven-zero products must be representable
    // (api_plan_schedule.inc:144-156)
    const uint64_t nonzero_a_rows = static_cast<uint64_t>(d.m) - s.zero_a_row_count;
    if (s.zero_a_row_count != 0 && static_cast<uint64_t>(d.n) > std::numeric_limits<uint64_t>::max() / s.zero_a_row_count)
      return RNS8_RANGE_ERROR;
    if (s.zero_b_col_count != 0 && nonzero_a_rows > std::numeric_limits<uint64_t>::max() / s.zero_b_col_count)
      return RNS8_RANGE_ERROR;
    s.zero_row_col_product_count =
        s.zero_a_row_count * static_cast<uint64_t>(d.n) + nonzero_a_rows * s.zero_b_col_count;
  }
  if (!d.tile_bounds || d.tile_bounds_count != count) return RNS8_INVALID_ARGUMENT;
  s.bounds.assign(d.tile_bounds, d.tile_bounds + count);
  const bool fixed = (d.flags & RNS8_PLAN_FORCE_FIXED_PREFIX) != 0;
  const bool zero_tiles = (d.flags & RNS8_PLAN_ALLOW_PROVEN_ZERO_TILE_SKIPS) != 0;
  uint32_t min_req = UINT32_MAX, max_req = 0, min_sel = UINT32_MAX, max_sel = 0;
  bool present[kMaxPrefix + 1] = {};
  s.entries.reserve(count);
  auto any_set = [](const std::vector<uint8_t>& mask, int64_t begin, int64_t end) {
    for (int64_t i = begin; i < end; ++i)
      if (mask[static_cast<std::size_t>(i)]) return true;
    return false;
  };
  for (uint64_t i = 0; i < count; ++i) {
    const uint64_t bound = s.bounds[i];
    if (d.semantics == RNS8_BOUNDED_I64 && bound > (uint64_t{1} << 63)) return RNS8_INVALID_ARGUMENT;
    const I256 range = tile_range(d.semantics, bound);
    const uint32_t bits = range.bit_length();
    const uint32_t req = required_prefix_for_range(range);
    if (req == 0 || req > budget) return RNS8_RANGE_ERROR;
    const uint32_t sel = fixed ? budget : req;
    min_req = std::min(min_req, req);
    max_req = std::max(max_req, req);
    min_sel = std::min(min_sel, sel);
    max_sel = std::max(max_sel, sel);
    s.range_bits = std::max(s.range_bits, bits);
    present[sel] = true;
    rns8_plan_tile_schedule_entry e = tile_entry(d.m, d.n, tm, tn, cols, i, req, sel, bits, 0);
    uint32_t f = zero_tiles && bound == 0 ? RNS8_TILE_SCHEDULE_ZERO_OUTPUT : 0u;
    if (proofs && (any_set(s.zero_a_rows, e.row_offset, e.row_offset + e.row_extent) ||
                   any_set(s.zero_b_cols, e.col_offset, e.col_offset + e.col_extent)))
      f |= RNS8_TILE_SCHEDULE_ZERO_ROW_COL_PRODUCT;
    e.flags = f;
    s.flags |= f;
    s.entries.push_back(e);
  }
  uint32_t rank[kMaxPrefix + 1] = {};
  for (uint32_t p = 0; p <= kMaxPrefix; ++p) {
    rank[p] = s.groups;
    s.groups += present[p] ? 1u : 0u;
  }
  for (auto& e : s.entries) e.group_index = rank[e.selected_prefix];
  s.min_required = count ? min_req : 0;
  s.max_required = max_req;
  s.min_selected = count ? min_sel : 0;
  s.max_selected = max_sel;
  s.adaptive_prefix = s.groups > 1 ? 1u : 0u;
  s.adaptive_skip = max_sel < budget ? 1u : 0u;
  if (s.groups == 1 && min_req == budget && max_req == budget && min_sel == budget && max_sel == budget &&
      s.flags == 0)
    s.entries.clear();  // every tile runs the plan prefix
  return RNS8_SUCCESS;
}

void plan_tile_entries(const rns8_plan& p, rns8_plan_tile_schedule_entry* out) {
  const bool crt = uses_rns_storage(p.desc.semantics);
  if (per_tile(p.desc.bound_kind) && !p.schedule.entries.empty()) {
    std::copy(p.schedule.entries.begin(), p.schedule.entries.end(), out);
    return;
  }
  for (uint64_t index = 0; index < p.tile_count; ++index) {
    if (per_tile(p.desc.bound_kind) && p.schedule.bounds.size() == p.tile_count) {
      const I256 range = tile_range(p.desc.semantics, p.schedule.bounds[index]);
      out[index] = tile_entry(p.desc.m, p.desc.n, p.desc.tile_m, p.desc.tile_n, p.tile_cols, index,
                              required_prefix_for_range(range), p.schedule.min_selected, range.bit_length(), 0);
      continue;
    }
    out[index] = tile_entry(p.desc.m, p.desc.n, p.desc.tile_m, p.desc.tile_n, p.tile_cols, index,
                            crt ? p.required_prefix : 0, crt ? p.prefix : 0, p.range_bits, 0);
  }
}

rns8_bound_kind storage_bound_kind(const rns8_plan& p) {
  if (p.desc.bound_kind != RNS8_BOUND_INPUT_RANGE_AND_K) return p.desc.bound_kind;
  return p.desc.semantics == RNS8_BOUNDED_I64 ? RNS8_BOUND_GLOBAL_MAX_ABS : RNS8_BOUND_GLOBAL_MAX_UNSIGNED;
}

// reference api_matrix_currentness_storage.inc:1-23
bool matrix_matches(const rns8_matrix& m, rns8_semantics s, rns8_bound_kind bk, int64_t rows, int64_t cols,
                    uint32_t prefix, uint32_t tile_m, uint32_t tile_n) {
  if (m.desc.semantics != s || m.desc.bound_kind != bk || m.desc.rows != rows || m.desc.cols != cols ||
      m.desc.logical_layout != RNS8_LAYOUT_ROW_MAJOR || m.desc.flags != 0)
    return false;
  // per-tile matrices carry the schedule's tile grid
  if (per_tile(bk) && (m.desc.tile_m != tile_m || m.desc.tile_n != tile_n)) return false;
  if (prefix == 0) return m.desc.max_prefix == 0;
  return m.prefix >= prefix && m.desc.max_prefix >= prefix;
}

}  // namespace rns8x

using namespace rns8x;

// ---- status and ladder queries ---------------------------------------------

const char* rns8_status_string(rns8_status status) {
  switch (status) {
    case RNS8_SUCCESS:
      return "success";
    case RNS8_INVALID_ARGUMENT:
      return "invalid argument";
    case RNS8_UNSUPPORTED_OS:
      return "unsupported operating system";
    case RNS8_UNSUPPORTED_ARCH:
      return "unsupported architecture";
    case RNS8_UNSUPPORTED_BACKEND:
      return "unsupported backend";
    case RNS8_RANGE_ERROR:
      return "range error";
    case RNS8_ACCUMULATION_OVERFLOW_RISK:
      return "accumulation overflow risk";
    case RNS8_WORKSPACE_TOO_SMALL:
      return "workspace too small";
    case RNS8_BACKEND_FAILURE:
      return "backend failure";
    case RNS8_VERIFICATION_FAILED:
      return "verification failed";
    case RNS8_INTERNAL_ERROR:
      return "internal error";
  }
  return "unknown status";
}

uint32_t rns8_default_modulus_count(void) { return kLadderSize; }

uint16_t rns8_default_modulus(uint32_t index) { return index < kLadderSize ? kLadder[index] : 0; }

double rns8_prefix_range_bits(uint32_t prefix) {
  if (prefix == 0 || prefix > kLadderSize) return 0.0;
  long double bits = 0.0L;
  for (uint32_t i = 0; i < prefix; ++i) bits += std::log2(static_cast<long double>(kLadder[i]));
  return static_cast<double>(bits);
}

rns8_status rns8_validate_default_moduli(void) {
  for (uint32_t i = 0; i < kLadderSize; ++i)
    for (uint32_t j = i + 1; j < kLadderSize; ++j) {
      uint32_t a = kLadder[i], b = kLadder[j];
      while (b) {
        const uint32_t t = a % b;
        a = b;
        b = t;
      }
      if (a != 1) return RNS8_INTERNAL_ERROR;
    }
  return RNS8_SUCCESS;
}

rns8_status rns8_mi355x_select_prefix(const rns8_gemm_desc* desc, uint32_t* out_prefix) {
  return guard([&]() -> rns8_status {
    if (!desc || !out_prefix) return RNS8_INVALID_ARGUMENT;
    // the whole of rns8_create_plan's validation, routing and schedule, so
    // the status is the one rns8_create_plan returns for this descriptor
    rns8_plan plan;
    const rns8_status st = init_plan(*desc, RNS8_BACKEND_HIP_DIRECT, plan);
    if (st != RNS8_SUCCESS) return st;
    *out_prefix = plan.prefix;
    return RNS8_SUCCESS;
  });
}

rns8_status rns8_mi355x_plan_schedule(const rns8_gemm_desc* desc, rns8_plan_schedule_info* info,
                                      rns8_plan_tile_schedule_entry* entries, uint64_t capacity, uint64_t* written) {
  return guard([&]() -> rns8_status {
    if (!desc || !info || !written) return RNS8_INVALID_ARGUMENT;
    rns8_plan plan;
    const rns8_status st = init_plan(*desc, RNS8_BACKEND_HIP_DIRECT, plan);
    if (st != RNS8_SUCCESS) return st;
    const rns8_status si = rns8_get_plan_schedule_info(&plan, info);
    if (si != RNS8_SUCCESS) return si;
    return rns8_get_plan_tile_schedule(&plan, entries, capacity, written);
  });
}

// ---- context -----------------------------------------------------------------

static void fill_device_info(rns8_context& ctx) {
  rns8_device_info& info = ctx.device_info;
  info = rns8_device_info{};
  info.struct_size = sizeof(info);
  info.abi_version = RNS8_ABI_VERSION;
  info.backend = RNS8_BACKEND_HIP_DIRECT;
  info.device_id = ctx.device_id;
  info.hip_available = 1;
  int rt = 0, drv = 0;
  (void)hipRuntimeGetVersion(&rt);
  (void)hipDriverGetVersion(&drv);
  info.hip_runtime_version = static_cast<uint32_t>(rt);
  info.hip_driver_version = static_cast<uint32_t>(drv);
  hipDeviceProp_t prop{};
  if (hipGetDeviceProperties(&prop, ctx.device_id) == hipSuccess) {
    info.global_mem_bytes = prop.totalGlobalMem;
    copy_text(info.name, sizeof(info.name), prop.name);
    copy_text(info.gcn_arch, sizeof(info.gcn_arch), prop.gcnArchName);
  }
  copy_text(info.detail, sizeof(info.detail),
            "rns8 MI355X: gfx950 int8 MFMA plane GEMM, HBM-resident residue planes, Garner export");
}

rns8_status rns8_create_context(int device_id, const rns8_context_options* options, rns8_context** out) {
  return guard([&]() -> rns8_status {
    if (!out) return RNS8_INVALID_ARGUMENT;
    *out = nullptr;
    if (options) {
      if (!valid_abi(options->struct_size, options->abi_version, sizeof(*options)) || options->flags != 0)
        return RNS8_INVALID_ARGUMENT;
      if (options->requested_backend != RNS8_BACKEND_AUTO && options->requested_backend != RNS8_BACKEND_HIP_DIRECT)
        return RNS8_UNSUPPORTED_BACKEND;
    }
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return RNS8_UNSUPPORTED_BACKEND;
    int dev = device_id;
    if (dev < 0) {
      if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    }
    if (dev >= count) return RNS8_INVALID_ARGUMENT;
    if (hipSetDevice(dev) != hipSuccess) return RNS8_BACKEND_FAILURE;
    hipDeviceProp_t prop{};
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return RNS8_BACKEND_FAILURE;
    // The kernels are built for gfx950 only.
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return RNS8_UNSUPPORTED_ARCH;
    // the device's address of the static scratch used by calls that allocate
    // nothing (rns8_mi355x_gemm_rns_noalloc); a failure here surfaces there
    (void)resolve_noalloc_scratch(dev);
    auto* ctx = new (std::nothrow) rns8_context();
    if (!ctx) return RNS8_INTERNAL_ERROR;
    ctx->device_id = dev;
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
      delete ctx;
      return RNS8_BACKEND_FAILURE;
    }
    fill_device_info(*ctx);
    *out = ctx;
    return RNS8_SUCCESS;
  });
}

rns8_status rns8_destroy_context(rns8_context* ctx) {
  return guard([&]() -> rns8_status {
    if (!ctx) return RNS8_SUCCESS;
    if (ctx->stream) {
      (void)hipSetDevice(ctx->device_id);
      (void)hipStreamSynchronize(ctx->stream);
    }
    release_oneshot_cache(*ctx);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return RNS8_SUCCESS;
  });
}

rns8_status rns8_get_device_info(rns8_context* ctx, rns8_device_info* out) {
  return guard([&]() -> rns8_status {
    if (!ctx || !out || !valid_abi(out->struct_size, out->abi_version, sizeof(*out))) return RNS8_INVALID_ARGUMENT;
    const uint64_t size = out->struct_size;
    const uint32_t version = out->abi_version;
    *out = ctx->device_info;
    out->struct_size = size;
    out->abi_version = version;
    return RNS8_SUCCESS;
  });
}

rns8_status rns8_get_backend_capability_info(rns8_backend_kind backend, rns8_backend_capability_info* out) {
  return guard([&]() -> rns8_status {
    if (!out || !valid_abi(out->struct_size, out->abi_version, sizeof(*out))) return RNS8_INVALID_ARGUMENT;
    if (static_cast<uint32_t>(backend) > static_cast<uint32_t>(RNS8_BACKEND_AMDGPU_BUILTINS))
      return RNS8_INVALID_ARGUMENT;
    reset_out(*out);
    out->backend = backend;
    const bool ours = backend == RNS8_BACKEND_HIP_DIRECT || backend == RNS8_BACKEND_AUTO;
    int count = 0;
    const bool hip = hipGetDeviceCount(&count) == hipSuccess && count > 0;
    out->is_accelerator = ours ? 1u : 0u;
    out->is_available = (ours && hip) ? 1u : 0u;
    out->is_matrix_engine_backend = ours ? 1u : 0u;
    out->supports_bounded_rns = ours ? 1u : 0u;
    out->supports_exact_wide_rns = ours ? 1u : 0u;
    out->supports_finite_u8 = ours ? 1u : 0u;
    out->compiled_kernel_available = ours ? 1u : 0u;
    out->exact_differential_validated = ours ? 1u : 0u;
    copy_text(out->backend_name, sizeof(out->backend_name), ours ? "hip_direct_gfx950" : "not_in_this_library");
    copy_text(out->selected_kernel, sizeof(out->selected_kernel),
              ours ? "plane_gemm_kernel<64> v_mfma_i32_32x32x32_i8" : "");
    copy_text(out->library_name, sizeof(out->library_name), "rns8_mi355x");
    copy_text(out->library_version, sizeof(out->library_version), "0.1");
    copy_text(out->epilogue_mode, sizeof(out->epilogue_mode), ours ? "in_register_centered_reduction" : "");
    copy_text(out->workspace_mode, sizeof(out->workspace_mode), ours ? "resident_planes_splitk_int8_residues" : "");
    copy_text(out->isa_evidence, sizeof(out->isa_evidence), ours ? "gfx950 v_mfma_i32_32x32x32_i8" : "");
    copy_text(out->status, sizeof(out->status), ours ? (hip ? "available" : "no_hip_device") : "unsupported_backend");
    copy_text(out->detail, sizeof(out->detail),
              ours ? "MI355X-native HIP_DIRECT implementation" : "backend not part of the MI355X library");
    return RNS8_SUCCESS;
  });
}

// ---- plan ----------------------------------------------------------------------

namespace rns8x {

// Plan state that needs no device: validation, prefix selection, tile grid,
// per-tile schedule, split-K sizing (reference api_plan_public_api.inc:3-73).
rns8_status init_plan(const rns8_gemm_desc& d, rns8_backend_kind backend, rns8_plan& plan) {
  if (!valid_abi(d.struct_size, d.abi_version, sizeof(d))) return RNS8_INVALID_ARGUMENT;
  const uint32_t budget0 = d.max_prefix == 0 ? default_prefix(d.semantics) : d.max_prefix;
  const rns8_status v = validate_gemm_desc(d, budget0);
  if (v != RNS8_SUCCESS) return v;
  // backend routing (reference api_plan_public_api.inc:19-33)
  if (d.requested_backend != RNS8_BACKEND_AUTO && d.requested_backend != backend) return RNS8_UNSUPPORTED_BACKEND;
  if (d.semantics == RNS8_WRAP_U64_MOD_2_64) return RNS8_UNSUPPORTED_BACKEND;
  uint32_t budget = 0, selected = 0, required = 0, bits = 0;
  uint64_t eff = 0;
  const rns8_status st = plan_prefix(d, budget, selected, required, bits, eff);
  if (st != RNS8_SUCCESS) return st;
  plan.desc = d;
  plan.desc.max_prefix = budget;
  plan.desc.bound = eff;
  if (plan.desc.tile_m == 0) plan.desc.tile_m = 128;
  if (plan.desc.tile_n == 0) plan.desc.tile_n = 128;
  plan.desc.tile_bounds = nullptr;
  plan.desc.zero_a_rows = nullptr;
  plan.desc.zero_b_cols = nullptr;
  plan.backend = backend;
  plan.budget = budget;
  plan.prefix = selected;
  plan.required_prefix = required;
  plan.range_bits = bits;
  plan.product = modulus_product(selected);
  plan.tile_rows = (static_cast<uint64_t>(d.m) + plan.desc.tile_m - 1) / plan.desc.tile_m;
  plan.tile_cols = (static_cast<uint64_t>(d.n) + plan.desc.tile_n - 1) / plan.desc.tile_n;
  plan.tile_count = plan.tile_rows * plan.tile_cols;
  if (per_tile(d.bound_kind)) {
    // copies the bounds and proof masks: the caller's arrays may change later
    const rns8_status ss = build_tile_schedule(d, budget, plan.schedule);
    if (ss != RNS8_SUCCESS) return ss;
    plan.desc.tile_bounds_count = plan.schedule.bounds.size();
    plan.desc.zero_a_rows_count = plan.schedule.zero_a_rows.size();
    plan.desc.zero_b_cols_count = plan.schedule.zero_b_cols.size();
  }
  const uint32_t planes = uses_finite_storage(d.semantics) ? 1u : selected;
  // Per-tile plans with a schedule run the tiled unit list (no K split). A
  // per-tile plan whose schedule collapsed (every tile at the budget) runs
  // the ordinary GEMM, so its K split and workspace are sized like a global
  // plan's: the skinny kernel splits K for long or narrow products.
  if (!per_tile(d.bound_kind) || plan.schedule.entries.empty()) {
    const GemmShape shape = choose_gemm_shape(d.m, d.n, d.k, planes);
    plan.splitk_slices = shape.slices;
    plan.splitk_bytes = shape.ws_bytes;
  }
  if (!per_tile(d.bound_kind)) {
    // the fused native-input GEMM shares the workspace
    if ((d.semantics == RNS8_BOUNDED_I64 || d.semantics == RNS8_BOUNDED_U64) &&
        choose_fused_shape(d.m, d.n, d.k, planes, padded_ld(d.n), plan.fused)) {
      plan.fused_ok = true;
      plan.splitk_bytes = std::max<uint64_t>(plan.splitk_bytes, plan.fused.ws_bytes);
    }
  }
  return RNS8_SUCCESS;
}

}  // namespace rns8x

rns8_status rns8_create_plan(rns8_context* ctx, const rns8_gemm_desc* desc, rns8_plan** out) {
  return guard([&]() -> rns8_status {
    if (!ctx || !desc || !out) return RNS8_INVALID_ARGUMENT;
    *out = nullptr;
    auto* plan = new (std::nothrow) rns8_plan();
    if (!plan) return RNS8_INTERNAL_ERROR;
    rns8_status st;
    try {
      st = init_plan(*desc, ctx->backend, *plan);
      plan->device_id = ctx->device_id;
      if (st == RNS8_SUCCESS && per_tile(plan->desc.bound_kind))
        st = hipSetDevice(ctx->device_id) == hipSuccess ? upload_tile_lists(*plan, ctx->stream) : RNS8_BACKEND_FAILURE;
    } catch (...) {
      free_tile_lists(*plan);
      delete plan;
      throw;
    }
    if (st != RNS8_SUCCESS) {
      free_tile_lists(*plan);
      delete plan;
      return st;
    }
    *out = plan;
    return RNS8_SUCCESS;
  });
}

rns8_status rns8_destroy_plan(rns8_plan* plan) {
  return guard([&]() -> rns8_status {
    if (!plan) return RNS8_SUCCESS;
    if (plan->units || plan->zero_fills || plan->export_tiles) {
      (void)hipSetDevice(plan->device_id);
      free_tile_lists(*plan);
    }
    delete plan;
    return RNS8_SUCCESS;
  });
}

// reference api_plan_contract_names.inc:39-51
static const char* bound_contract_name(const rns8_plan& p) {
  if (p.desc.bound_kind == RNS8_BOUND_INPUT_RANGE_AND_K) return "input_range_and_k_derived_output_bound";
  if (per_tile(p.desc.bound_kind)) return "per_tile_output_bounds";
  if (p.desc.bound_kind == RNS8_BOUND_GLOBAL_MAX_ABS || p.desc.bound_kind == RNS8_BOUND_GLOBAL_MAX_UNSIGNED)
    return "global_output_bound";
  return "not_applicable";
}

rns8_status rns8_get_plan_schedule_info(const rns8_plan* plan, rns8_plan_schedule_info* out) {
  return guard([&]() -> rns8_status {
    if (!plan || !out || !valid_abi(out->struct_size, out->abi_version, sizeof(*out))) return RNS8_INVALID_ARGUMENT;
    reset_out(*out);
    out->tile_m = plan->desc.tile_m;
    out->tile_n = plan->desc.tile_n;
    out->tile_rows = plan->tile_rows;
    out->tile_cols = plan->tile_cols;
    out->tile_count = plan->tile_count;
    const bool crt = uses_rns_storage(plan->desc.semantics);
    if (per_tile(plan->desc.bound_kind)) {
      const TileSchedule& sc = plan->schedule;
      out->min_required_prefix = sc.min_required;
      out->max_required_prefix = sc.max_required;
      out->min_selected_prefix = sc.min_selected;
      out->max_selected_prefix = sc.max_selected;
      out->prefix_group_count = sc.groups;
      out->adaptive_prefix_active = sc.adaptive_prefix;
      out->adaptive_skip_active = sc.adaptive_skip;
      out->range_bit_length = sc.range_bits;
      out->flags = sc.flags;
      out->zero_a_row_count = sc.zero_a_row_count;
      out->zero_b_col_count = sc.zero_b_col_count;
      out->zero_row_col_product_count = sc.zero_row_col_product_count;
    } else {
      out->min_required_prefix = crt ? plan->required_prefix : 0;
      out->max_required_prefix = crt ? plan->required_prefix : 0;
      out->min_selected_prefix = crt ? plan->prefix : 0;
      out->max_selected_prefix = crt ? plan->prefix : 0;
      out->prefix_group_count = crt ? 1u : 0u;
      out->adaptive_prefix_active = 0;
      out->adaptive_skip_active = (crt && plan->prefix < plan->budget) ? 1u : 0u;
      out->range_bit_length = plan->range_bits;
      out->flags = 0;
    }
    out->bound_kind = plan->desc.bound_kind;
    out->effective_bound = plan->desc.bound;
    out->lhs_bound = plan->desc.lhs_bound;
    out->rhs_bound = plan->desc.rhs_bound;
    copy_text(out->bound_contract, sizeof(out->bound_contract), bound_contract_name(*plan));
    return RNS8_SUCCESS;
  });
}

rns8_status rns8_get_plan_tile_schedule(const rns8_plan* plan, rns8_plan_tile_schedule_entry* entries,
                                        uint64_t capacity, uint64_t* written) {
  return guard([&]() -> rns8_status {
    if (!plan || !written) return RNS8_INVALID_ARGUMENT;
    *written = plan->tile_count;
    if (!entries || capacity == 0) return RNS8_SUCCESS;
    if (capacity < plan->tile_count) return RNS8_WORKSPACE_TOO_SMALL;
    plan_tile_entries(*plan, entries);
    return RNS8_SUCCESS;
  });
}

rns8_status rns8_get_plan_backend_info(const rns8_plan* plan, rns8_plan_backend_info* out) {
  return guard([&]() -> rns8_status {
    if (!plan || !out || !valid_abi(out->struct_size, out->abi_version, sizeof(*out))) return RNS8_INVALID_ARGUMENT;
    reset_out(*out);
    out->backend = plan->backend;
    out->is_accelerator = 1;
    out->is_matrix_engine_backend = 1;
    out->compiled_kernel_available = 1;
    out->exact_differential_validated = 1;
    out->workspace_required_bytes = plan->splitk_bytes;
    const bool listed = per_tile(plan->desc.bound_kind) && !plan->schedule.entries.empty();
    const uint32_t planes = uses_finite_storage(plan->desc.semantics) ? 1u : (plan->prefix ? plan->prefix : 1u);
    const GemmShape shape = choose_gemm_shape(plan->desc.m, plan->desc.n, plan->desc.k, planes);
    const bool skinny = !listed && shape.tile == 16;
    copy_text(out->selected_kernel, sizeof(out->selected_kernel),
              listed ? (plan->unit_edge == 256 ? "plane_gemm_kernel listed 256x256 units (per-tile schedule)"
                                               : "plane_gemm_kernel listed 128x128 units (per-tile schedule)")
              : skinny ? (shape.slices > 1 ? "skinny_gemm_kernel 16-column rows, K split + residue_finalize_kernel"
                                           : "skinny_gemm_kernel 16-column rows")
              : shape.slices > 1 ? "plane_gemm_kernel 128x128 K split + residue_finalize_kernel"
              : shape.tile == 256 ? "plane_gemm_kernel 256x256 tile, 4-stage LDS DMA ring"
                                  : "plane_gemm_kernel 128x128 tile, 4-stage LDS DMA ring");
    copy_text(out->accelerator_library, sizeof(out->accelerator_library), "none (hand-written HIP)");
    copy_text(out->capability_status, sizeof(out->capability_status), "available");
    copy_text(out->epilogue_mode, sizeof(out->epilogue_mode), "in_register_centered_reduction");
    copy_text(out->workspace_mode, sizeof(out->workspace_mode),
              plan->splitk_slices > 1 ? "splitk_int8_residues" : "none");
    copy_text(out->isa_evidence, sizeof(out->isa_evidence),
              skinny ? "gfx950 v_mfma_i32_16x16x64_i8" : "gfx950 v_mfma_i32_32x32x32_i8");
    out->accumulator_k_block_size = static_cast<uint64_t>(plan->desc.k < kSafeKBlock ? plan->desc.k : kSafeKBlock);
    out->accumulator_k_block_cap = static_cast<uint64_t>(kSafeKBlock);
    out->accumulator_modulus = uses_finite_storage(plan->desc.semantics) ? plan->desc.finite_modulus : 0;
    out->accumulator_max_lhs_abs = 128;
    out->accumulator_max_rhs_abs = 128;
    out->accumulator_max_product = 16384;
    out->accumulator_uses_int32_inner_product = 1;
    out->accumulator_safe_for_k_block = 1;
    copy_text(out->accumulator_input_domain, sizeof(out->accumulator_input_domain), "centered_int8_residue");
    copy_text(out->accumulator_signedness, sizeof(out->accumulator_signedness), "signed");
    copy_text(out->accumulator_type, sizeof(out->accumulator_type), "int32");
    copy_text(out->accumulator_modulus_policy, sizeof(out->accumulator_modulus_policy),
              "reduce_to_centered_every_65536_k");
    copy_text(out->accumulator_safety_status, sizeof(out->accumulator_safety_status), "safe");
    return RNS8_SUCCESS;
  });
}

rns8_status rns8_get_plan_packing_info(const rns8_plan* plan, rns8_plan_packing_info* out) {
  return guard([&]() -> rns8_status {
    if (!plan || !out || !valid_abi(out->struct_size, out->abi_version, sizeof(*out))) return RNS8_INVALID_ARGUMENT;
    reset_out(*out);
    out->backend = plan->backend;
    out->semantics = plan->desc.semantics;
    out->uses_resident_matrix_inputs = 1;
    out->uses_matrix_engine_pack_layout = 1;
    out->flags = RNS8_PLAN_PACKING_SOURCE_VERSIONED_INPUTS | RNS8_PLAN_PACKING_SAME_SOURCE_VERSION_PACK_ELISION;
    const bool finite = uses_finite_storage(plan->desc.semantics);
    out->input_domain = finite ? RNS8_OUTPUT_DOMAIN_FINITE_U8 : RNS8_OUTPUT_DOMAIN_RNS_RESIDUE;
    out->output_domain = finite ? RNS8_OUTPUT_DOMAIN_FINITE_U8 : RNS8_OUTPUT_DOMAIN_RNS_RESIDUE;
    out->output_device_current = 1;
    out->next_op_flags = RNS8_NEXT_OP_FINAL_EXPORT | RNS8_NEXT_OP_RNS_GEMM;
    out->accumulator_workspace_bytes = plan->splitk_bytes;
    out->total_transient_workspace_bytes = plan->splitk_bytes;
    copy_text(out->input_domain_name, sizeof(out->input_domain_name), finite ? "finite_u8" : "rns_residue");
    copy_text(out->output_domain_name, sizeof(out->output_domain_name), finite ? "finite_u8" : "rns_residue");
    copy_text(out->next_op_hint, sizeof(out->next_op_hint), "export or chain into rns8_gemm_rns");
    copy_text(out->a_layout_version, sizeof(out->a_layout_version), "rns8_mi355x_planes_v1");
    copy_text(out->b_layout_version, sizeof(out->b_layout_version), "rns8_mi355x_planes_v1");
    copy_text(out->output_layout_version, sizeof(out->output_layout_version), "rns8_mi355x_planes_v1");
    copy_text(out->detail, sizeof(out->detail),
              "planes row-major int8, rows padded to 16 bytes, planes to 256 bytes; B transposed in LDS");
    return RNS8_SUCCESS;
  });
}

// reference api_plan_public_api.inc:255-368: the contract rns8_gemm_rns_grouped
// and rns8_gemm_finite_u8_grouped enforce for this plan. The flags and the
// policy names that describe the caller-visible contract are the reference's;
// the layout and descriptor policies name this implementation's.
rns8_status rns8_get_grouped_dispatch_contract_info(const rns8_plan* plan, uint32_t task_count,
                                                    rns8_grouped_dispatch_contract_info* out) {
  return guard([&]() -> rns8_status {
    if (!plan || !out || !valid_abi(out->struct_size, out->abi_version, sizeof(*out))) return RNS8_INVALID_ARGUMENT;
    reset_out(*out);
    out->backend = plan->backend;
    out->semantics = plan->desc.semantics;
    out->task_count = task_count;
    out->same_shape_required = 1;
    out->same_semantics_required = 1;
    out->compact_row_major_required = 1;
    out->unique_matrix_handles_required = 1;
    out->unique_workspace_handles_required = 1;
    out->same_plan_fingerprint_required = 1;
    out->same_device_required = 1;
    out->device_resident_inputs_required = 1;
    out->per_task_source_versions_required = 1;
    out->produces_device_current_output = 1;
    out->final_export_required_for_host_output = 1;
    out->per_task_status_required = 1;
    out->checksum_policy_required = 1;
    out->descriptor_reuse_validated = 1;
    out->flags = RNS8_GROUPED_DISPATCH_CONTRACT_SAME_SHAPE_REQUIRED |
                 RNS8_GROUPED_DISPATCH_CONTRACT_COMPACT_ROW_MAJOR_REQUIRED |
                 RNS8_GROUPED_DISPATCH_CONTRACT_UNIQUE_TASK_HANDLES_REQUIRED |
                 RNS8_GROUPED_DISPATCH_CONTRACT_ONE_WORKSPACE_PER_TASK_REQUIRED |
                 RNS8_GROUPED_DISPATCH_CONTRACT_SAME_DEVICE_REQUIRED |
                 RNS8_GROUPED_DISPATCH_CONTRACT_PER_TASK_SOURCE_VERSION_REQUIRED |
                 RNS8_GROUPED_DISPATCH_CONTRACT_DEVICE_CURRENT_OUTPUT_REQUIRED |
                 RNS8_GROUPED_DISPATCH_CONTRACT_PUBLIC_PACK_EXPLICIT |
                 RNS8_GROUPED_DISPATCH_CONTRACT_PUBLIC_EXPORT_EXPLICIT |
                 RNS8_GROUPED_DISPATCH_CONTRACT_GENERIC_BUCKETING_UNAVAILABLE |
                 RNS8_GROUPED_DISPATCH_CONTRACT_AUTO_ROUTING_DISABLED;
    copy_text(out->descriptor_layout, sizeof(out->descriptor_layout), "same_shape_resident_task_triplets_v1");
    copy_text(out->bucket_policy, sizeof(out->bucket_policy), "single_same_shape_bucket");
    copy_text(out->source_version_policy, sizeof(out->source_version_policy),
              "per_task_monotonic_source_version_repack");
    copy_text(out->workspace_policy, sizeof(out->workspace_policy), "one_workspace_per_task_shared_plan");
    copy_text(out->matrix_ownership_policy, sizeof(out->matrix_ownership_policy),
              "caller_owns_unique_task_triplets_until_grouped_call_returns");
    copy_text(out->descriptor_reuse_policy, sizeof(out->descriptor_reuse_policy),
              "reuse_after_shape_workspace_source_validation");
    copy_text(out->stride_policy, sizeof(out->stride_policy), "matrix_ld_matches_logical_shape_host_output_ld_explicit");
    copy_text(out->output_currentness_policy, sizeof(out->output_currentness_policy),
              "device_residue_current_after_grouped_gemm_host_output_after_export");
    copy_text(out->lifetime_policy, sizeof(out->lifetime_policy),
              "task_matrices_and_workspaces_valid_until_grouped_call_returns");
    copy_text(out->checksum_policy, sizeof(out->checksum_policy), "combined_per_task_checksum_u64");
    copy_text(out->status_policy, sizeof(out->status_policy), "fail_fast_per_task_operation_status");
    copy_text(out->device_descriptor_policy, sizeof(out->device_descriptor_policy),
              "task_pointer_table_in_kernel_arguments_32_per_launch");
    const rns8_semantics s = plan->desc.semantics;
    const char* domain = s == RNS8_BOUNDED_I64 || s == RNS8_BOUNDED_U64       ? "native_i64_u64_host"
                         : s == RNS8_EXACT_WIDE_SIGNED || s == RNS8_EXACT_WIDE_UNSIGNED ? "exact_wide_limb_host"
                         : s == RNS8_FINITE_FIELD_U8 || s == RNS8_FINITE_RING_U8       ? "finite_u8_host"
                                                                                       : "wrap64_u64_host";
    copy_text(out->output_domain, sizeof(out->output_domain), domain);
    const char* reason = nullptr;
    if (plan->backend != RNS8_BACKEND_HIP_DIRECT) reason = "backend_not_hip_direct";
    else if (task_count <= 1) reason = "task_count_must_exceed_one";
    else if (s == RNS8_WRAP_U64_MOD_2_64) reason = "unsupported_grouped_semantics";
    else if (plan->desc.m <= 0 || plan->desc.n <= 0 || plan->desc.k <= 0) reason = "invalid_plan_shape";
    if (reason) {
      copy_text(out->unsupported_reason, sizeof(out->unsupported_reason), reason);
      out->flags |= RNS8_GROUPED_DISPATCH_CONTRACT_BENCHMARK_ONLY_EXECUTION;
      copy_text(out->detail, sizeof(out->detail), "grouped execution is not available for this plan and task count");
    } else {
      out->descriptor_contract_supported = 1;
      out->public_execution_available = 1;
      copy_text(out->detail, sizeof(out->detail),
                "one persistent gfx950 launch per 65536-K block covers up to 32 tasks (task-major unit order); "
                "inputs are packed before the call and outputs exported after it");
    }
    return RNS8_SUCCESS;
  });
}

// ---- workspace ---------------------------------------------------------------------

rns8_status rns8_create_workspace(rns8_context* ctx, const rns8_plan* plan, rns8_workspace** out) {
  return guard([&]() -> rns8_status {
    if (!ctx || !plan || !out) return RNS8_INVALID_ARGUMENT;
    *out = nullptr;
    if (plan->backend != ctx->backend || plan->device_id != ctx->device_id) return RNS8_INVALID_ARGUMENT;
    auto* ws = new (std::nothrow) rns8_workspace();
    if (!ws) return RNS8_INTERNAL_ERROR;
    ws->backend = plan->backend;
    ws->semantics = plan->desc.semantics;
    ws->bound_kind = plan->desc.bound_kind;
    ws->m = plan->desc.m;
    ws->n = plan->desc.n;
    ws->k = plan->desc.k;
    ws->prefix = plan->prefix;
    ws->finite_modulus = plan->desc.finite_modulus;
    ws->device_id = ctx->device_id;
    if (plan->splitk_bytes) {
      if (hipSetDevice(ctx->device_id) != hipSuccess ||
          hipMalloc(reinterpret_cast<void**>(&ws->splitk), plan->splitk_bytes) != hipSuccess) {
        delete ws;
        return RNS8_BACKEND_FAILURE;
      }
      ws->splitk_bytes = plan->splitk_bytes;
      // zeroed once; every launch that uses it writes each cell it later reads
      if (launch_zero_words(reinterpret_cast<uint32_t*>(ws->splitk), plan->splitk_bytes / 4, ctx->stream) !=
              hipSuccess ||
          hipStreamSynchronize(ctx->stream) != hipSuccess) {
        free_device(ws->splitk);
        delete ws;
        return RNS8_BACKEND_FAILURE;
      }
    }
    *out = ws;
    return RNS8_SUCCESS;
  });
}

rns8_status rns8_destroy_workspace(rns8_workspace* workspace) {
  return guard([&]() -> rns8_status {
    if (!workspace) return RNS8_SUCCESS;
    if (workspace->splitk) {
      (void)hipSetDevice(workspace->device_id);
      free_device(workspace->splitk);
    }
    delete workspace;
    return RNS8_SUCCESS;
  });
}

// ---- matrix ------------------------------------------------------------------------

rns8_status rns8_create_matrix(rns8_context* ctx, const rns8_matrix_desc* desc, rns8_matrix** out) {
  return guard([&]() -> rns8_status {
    static std::atomic<uint64_t> next_id{1};
    if (!ctx || !desc || !out) return RNS8_INVALID_ARGUMENT;
    *out = nullptr;
    rns8_matrix layout;
    const rns8_status v = init_matrix(*desc, ctx->backend, ctx->device_id, layout);
    if (v != RNS8_SUCCESS) return v;
    auto* m = new (std::nothrow) rns8_matrix();
    if (!m) return RNS8_INTERNAL_ERROR;
    m->desc = layout.desc;
    m->backend = layout.backend;
    m->device_id = layout.device_id;
    m->instance_id = next_id.fetch_add(1);
    m->prefix = layout.prefix;
    m->plane_ld = layout.plane_ld;
    m->plane_pitch = layout.plane_pitch;
    m->plane_bytes = layout.plane_bytes;
    if (hipSetDevice(ctx->device_id) != hipSuccess ||
        hipMalloc(reinterpret_cast<void**>(&m->planes), m->plane_bytes) != hipSuccess) {
      delete m;
      return RNS8_BACKEND_FAILURE;
    }
    // exact-wide matrices: the device proof (two sets of axis records and the
    // pack accumulators, zeroed below with the planes) and its event
    const uint64_t proof_bytes = rns8_matrix::proof_bytes(m->desc.rows, m->desc.cols);
    if (exact_wide(desc->semantics) &&
        (hipMalloc(reinterpret_cast<void**>(&m->proof_device), proof_bytes) != hipSuccess ||
         hipEventCreateWithFlags(&m->proof_event, hipEventDisableTiming) != hipSuccess)) {
      free_device(m->planes);
      free_device(m->proof_device);
      delete m;
      return RNS8_BACKEND_FAILURE;
    }
    // zero planes: a fresh matrix holds the integer 0 and keeps padding zero
    if (launch_zero_words(reinterpret_cast<uint32_t*>(m->planes), m->plane_bytes / 4, ctx->stream) != hipSuccess ||
        (m->proof_device &&
         launch_zero_words(reinterpret_cast<uint32_t*>(m->proof_device), proof_bytes / 4, ctx->stream) !=
             hipSuccess) ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) {
      free_device(m->planes);
      free_device(m->proof_device);
      if (m->proof_event) (void)hipEventDestroy(m->proof_event);
      delete m;
      return RNS8_BACKEND_FAILURE;
    }
    // nothing current until a pack or a GEMM writes the planes (reference
    // internal.hpp:106): a GEMM on a never-packed operand and an export of a
    // never-computed result are refused with RNS8_INVALID_ARGUMENT
    m->device_current = false;
    *out = m;
    return RNS8_SUCCESS;
  });
}

rns8_status rns8_destroy_matrix(rns8_matrix* matrix) {
  return guard([&]() -> rns8_status {
    if (!matrix) return RNS8_SUCCESS;
    (void)hipSetDevice(matrix->device_id);
    free_device(matrix->planes);
    free_device(matrix->upload);
    free_device(matrix->staging);
    free_device(matrix->status);
    free_device(matrix->proof_device);
    if (matrix->proof_event) (void)hipEventDestroy(matrix->proof_event);
    delete matrix;
    return RNS8_SUCCESS;
  });
}

rns8_status rns8_get_matrix_storage_info(const rns8_matrix* matrix, rns8_matrix_storage_info* out) {
  return guard([&]() -> rns8_status {
    if (!matrix || !out || !valid_abi(out->struct_size, out->abi_version, sizeof(*out))) return RNS8_INVALID_ARGUMENT;
    reset_out(*out);
    out->backend = matrix->backend;
    out->semantics = matrix->desc.semantics;
    out->logical_layout = matrix->desc.logical_layout;
    out->bound_kind = matrix->desc.bound_kind;
    out->rows = matrix->desc.rows;
    out->cols = matrix->desc.cols;
    out->logical_ld = matrix->desc.logical_ld;
    out->max_prefix = matrix->desc.max_prefix;
    out->finite_modulus = matrix->finite_modulus;
    out->matrix_instance_id = matrix->instance_id;
    out->source_version = matrix->source_version;
    out->device_residues_current = matrix->device_current ? 1u : 0u;
    out->uses_residue_storage = 1;
    out->hip_device_id = matrix->device_id;
    out->device_residue_bytes = matrix->plane_bytes;
    copy_text(out->layout_version, sizeof(out->layout_version), "rns8_mi355x_planes_v1");
    copy_text(out->storage_scope, sizeof(out->storage_scope), "device_only");
    copy_text(out->detail, sizeof(out->detail), "modulus-major centered int8 planes in HBM; no host mirror");
    return RNS8_SUCCESS;
  });
}

rns8_status rns8_mi355x_get_matrix_planes(const rns8_matrix* matrix, void** d_planes, int64_t* row_pitch,
                                          int64_t* plane_pitch_out, uint32_t* plane_count) {
  return guard([&]() -> rns8_status {
    if (!matrix || !d_planes || !row_pitch || !plane_pitch_out || !plane_count) return RNS8_INVALID_ARGUMENT;
    *d_planes = matrix->planes;
    *row_pitch = matrix->plane_ld;
    *plane_pitch_out = matrix->plane_pitch;
    *plane_count = matrix->prefix;
    return RNS8_SUCCESS;
  });
}

rns8_status rns8_get_resident_lifetime_info(const rns8_matrix* matrix, const rns8_plan* plan,
                                            const rns8_workspace* workspace, rns8_resident_matrix_role role,
                                            rns8_resident_lifetime_info* out) {
  return guard([&]() -> rns8_status {
    if (!matrix || !out || !valid_abi(out->struct_size, out->abi_version, sizeof(*out))) return RNS8_INVALID_ARGUMENT;
    if (workspace && !plan) return RNS8_INVALID_ARGUMENT;
    if (static_cast<uint32_t>(role) > static_cast<uint32_t>(RNS8_RESIDENT_MATRIX_ROLE_C)) return RNS8_INVALID_ARGUMENT;
    reset_out(*out);
    out->backend = matrix->backend;
    out->semantics = matrix->desc.semantics;
    out->logical_layout = matrix->desc.logical_layout;
    out->bound_kind = matrix->desc.bound_kind;
    out->matrix_role = role;
    out->current_output_domain =
        uses_finite_storage(matrix->desc.semantics) ? RNS8_OUTPUT_DOMAIN_FINITE_U8 : RNS8_OUTPUT_DOMAIN_RNS_RESIDUE;
    out->rows = matrix->desc.rows;
    out->cols = matrix->desc.cols;
    out->logical_ld = matrix->desc.logical_ld;
    out->max_prefix = matrix->desc.max_prefix;
    out->finite_modulus = matrix->finite_modulus;
    out->source_version = matrix->source_version;
    out->hip_device_id = matrix->device_id;
    out->source_version_valid = matrix->source_version != 0 ? 1u : 0u;
    out->device_current = matrix->device_current ? 1u : 0u;
    out->device_resident = 1;
    out->plan_binding_available = plan ? 1u : 0u;
    if (plan) {
      const bool rows_ok = role == RNS8_RESIDENT_MATRIX_ROLE_B ? matrix->desc.rows == plan->desc.k
                                                                : matrix->desc.rows == plan->desc.m;
      const bool cols_ok = role == RNS8_RESIDENT_MATRIX_ROLE_A ? matrix->desc.cols == plan->desc.k
                                                                : matrix->desc.cols == plan->desc.n;
      out->plan_binding_matches =
          (matrix->desc.semantics == plan->desc.semantics && rows_ok && cols_ok) ? 1u : 0u;
    }
    out->workspace_binding_available = workspace ? 1u : 0u;
    if (workspace && plan) {
      out->workspace_identity_matches = (workspace->m == plan->desc.m && workspace->n == plan->desc.n &&
                                         workspace->k == plan->desc.k && workspace->prefix == plan->prefix)
                                            ? 1u
                                            : 0u;
      out->workspace_schedule_matches = out->workspace_identity_matches;
      out->workspace_backend_matches = workspace->backend == plan->backend ? 1u : 0u;
      out->workspace_binding_matches = out->workspace_identity_matches & out->workspace_backend_matches;
    }
    out->device_id_matches = 1;
    out->can_feed_rns_gemm = (matrix->device_current && uses_rns_storage(matrix->desc.semantics)) ? 1u : 0u;
    out->can_feed_final_export = matrix->device_current ? 1u : 0u;
    copy_text(out->current_domain, sizeof(out->current_domain),
              uses_finite_storage(matrix->desc.semantics) ? "finite_u8" : "rns_residue");
    static const char* const names[] = {"unknown", "a", "b", "c"};
    copy_text(out->matrix_role_name, sizeof(out->matrix_role_name), names[static_cast<uint32_t>(role)]);
    copy_text(out->source_version_policy, sizeof(out->source_version_policy), "same_nonzero_version_elides_pack");
    copy_text(out->lifetime_policy, sizeof(out->lifetime_policy), "device_planes_live_until_destroy");
    return RNS8_SUCCESS;
  });
}
