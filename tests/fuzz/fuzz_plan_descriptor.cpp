// libFuzzer target over the device-free planning entries, built with
// AddressSanitizer and UndefinedBehaviorSanitizer (tests/fuzz/Makefile).
// After the reference's tests/fuzz/rns8_fuzz_plan_descriptor.cpp (built by
// cmake/rns8_targets.cmake:229-237), which drives rns8_create_plan on its CPU
// backend; here the same validation, prefix selection and tile schedule run
// through rns8_mi355x_select_prefix and rns8_mi355x_plan_schedule, which need
// no device.
//
// The input decodes into a gemm descriptor whose every scalar field takes
// full-range values (dimensions, tile sizes, bounds, prefixes, flags,
// semantics and bound kinds, including values outside their enums), plus
// per-tile bound and zero-mask arrays of up to 256 entries whose declared
// counts always match their storage (the counts are the caller's promise
// about its own arrays). Checked on every input, beyond the sanitizers:
//   * both entries return a status the API defines;
//   * select_prefix and plan_schedule agree on success, and on the prefix;
//   * a successful schedule reports tile_count = tile_rows * tile_cols and
//     min <= max for the required and selected prefixes (all <= 20);
//   * entries are only written within the caller's capacity, and each entry
//     lies inside the m x n output.
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "rns8/rns8.h"
#include "rns8_mi355x.h"

namespace {

struct Reader {
  const uint8_t* p;
  const uint8_t* end;
  uint64_t u64() {
    uint64_t v = 0;
    for (int i = 0; i < 8 && p < end; ++i) v |= static_cast<uint64_t>(*p++) << (8 * i);
    return v;
  }
  uint32_t u32() { return static_cast<uint32_t>(u64()); }
  uint8_t u8() { return p < end ? *p++ : 0; }
};

// a dimension: mostly small, sometimes at the edges of int64
int64_t dim(Reader& r) {
  const uint8_t sel = r.u8();
  const uint64_t v = r.u64();
  switch (sel % 8) {
    case 0: return static_cast<int64_t>(v);
    case 1: return -static_cast<int64_t>(v % 4);
    case 2: return INT64_MAX - static_cast<int64_t>(v % 4);
    case 3: return static_cast<int64_t>(v % (uint64_t{1} << 40));
    default: return static_cast<int64_t>(v % 1024) + 1;
  }
}

uint32_t tile(Reader& r) {
  static const uint32_t kTiles[] = {0, 64, 128, 256, 512, 32, 96, 1024};
  const uint8_t sel = r.u8();
  return sel < 200 ? kTiles[sel % 8] : r.u32();
}

void fail(const char* what, long long a = 0, long long b = 0) {
  std::fprintf(stderr, "FUZZ CHECK FAILED: %s (%lld, %lld)\n", what, a, b);
  std::abort();
}

bool known_status(rns8_status s) { return static_cast<uint32_t>(s) <= RNS8_INTERNAL_ERROR; }

}  // namespace

extern "C" int LLVMFuzzerTestOneInput(const uint8_t* data, std::size_t size) {
  Reader r{data, data + size};
  rns8_gemm_desc d;
  std::memset(&d, 0, sizeof(d));
  const uint8_t header = r.u8();
  d.struct_size = header & 1 ? r.u64() : sizeof(d);
  d.abi_version = header & 2 ? r.u32() : RNS8_ABI_VERSION;
  d.semantics = static_cast<rns8_semantics>(r.u8() % 9);
  d.bound_kind = static_cast<rns8_bound_kind>(r.u8() % 7);
  d.requested_backend = static_cast<rns8_backend_kind>(r.u8() % 8);
  d.m = dim(r);
  d.n = dim(r);
  d.k = dim(r);
  const uint8_t bsel = r.u8();
  d.bound = bsel % 4 == 0 ? r.u64() : bsel % 4 == 1 ? (r.u64() % 4096) : bsel % 4 == 2 ? UINT64_MAX - r.u8() : 0;
  d.max_prefix = r.u8() % 24;
  d.tile_m = tile(r);
  d.tile_n = tile(r);
  d.finite_modulus = r.u8() % 4 == 0 ? r.u32() : r.u8() + 1u;
  d.flags = r.u8() % 4 == 0 ? r.u32() : r.u8() & 7u;
  d.lhs_bound = header & 4 ? r.u64() : 0;
  d.rhs_bound = header & 8 ? r.u64() : 0;

  std::vector<uint64_t> bounds;
  std::vector<uint8_t> zero_a, zero_b;
  if (header & 16) {
    bounds.resize(r.u8());
    for (auto& b : bounds) b = r.u8() % 2 ? r.u64() : r.u8();
    d.tile_bounds = bounds.empty() ? nullptr : bounds.data();
    d.tile_bounds_count = bounds.size();
  }
  if (header & 32) {
    zero_a.resize(r.u8());
    for (auto& z : zero_a) z = r.u8() & 1;
    zero_b.resize(r.u8());
    for (auto& z : zero_b) z = r.u8() & 1;
    d.zero_a_rows = zero_a.empty() ? nullptr : zero_a.data();
    d.zero_a_rows_count = zero_a.size();
    d.zero_b_cols = zero_b.empty() ? nullptr : zero_b.data();
    d.zero_b_cols_count = zero_b.size();
  }

  uint32_t prefix = 0xFFFFFFFFu;
  const rns8_status sp = rns8_mi355x_select_prefix(&d, &prefix);
  if (!known_status(sp)) fail("select_prefix status");

  rns8_plan_schedule_info info;
  std::memset(&info, 0, sizeof(info));
  info.struct_size = sizeof(info);
  info.abi_version = RNS8_ABI_VERSION;
  const uint64_t capacity = r.u8() % 64;
  // one guard entry past the capacity must stay untouched
  std::vector<rns8_plan_tile_schedule_entry> entries(capacity + 1);
  std::memset(entries.data(), 0xA5, entries.size() * sizeof(entries[0]));
  uint64_t written = 0;
  const rns8_status ss =
      rns8_mi355x_plan_schedule(&d, &info, capacity ? entries.data() : nullptr, capacity, &written);
  if (!known_status(ss)) fail("plan_schedule status");
  if ((sp == RNS8_SUCCESS) != (ss == RNS8_SUCCESS || ss == RNS8_WORKSPACE_TOO_SMALL)) fail("entries disagree", sp, ss);
  {
    const auto* guard = reinterpret_cast<const uint8_t*>(&entries[capacity]);
    for (std::size_t i = 0; i < sizeof(entries[0]); ++i)
      if (guard[i] != 0xA5) fail("entry written past the capacity");
  }
  if (ss == RNS8_SUCCESS || ss == RNS8_WORKSPACE_TOO_SMALL) {
    if (written != info.tile_count) fail("written count");
    if (info.tile_count != info.tile_rows * info.tile_cols) fail("tile count");
    if (info.min_required_prefix > info.max_required_prefix || info.min_selected_prefix > info.max_selected_prefix)
      fail("prefix order");
    if (info.max_required_prefix > 20 || info.max_selected_prefix > 20) fail("prefix range");
    if (info.max_selected_prefix != 0 && prefix != info.max_selected_prefix && !(d.bound_kind == RNS8_BOUND_PER_TILE_MAX_ABS || d.bound_kind == RNS8_BOUND_PER_TILE_MAX_UNSIGNED))
      fail("prefix disagrees");
  }
  if (ss == RNS8_SUCCESS && capacity >= info.tile_count) {
    for (uint64_t t = 0; t < info.tile_count; ++t) {
      const auto& e = entries[t];
      if (e.row_offset < 0 || e.col_offset < 0 || e.row_extent <= 0 || e.col_extent <= 0 ||
          e.row_offset + e.row_extent > d.m || e.col_offset + e.col_extent > d.n)
        fail("entry outside the output");
    }
  }
  return 0;
}
