// Device lists of a per-tile bounded plan, built once when the plan is created.
//
// GEMM (reference cpu_reference.cpp:231-257, the GEMM over a tile schedule):
// planes [0, selected) of every tile are computed, zero-output tiles get 0 in
// those planes, and planes from a tile's selected prefix up are left as they
// are. The listed GEMM runs output tiles of one plane (256 x 256, or 128 x 128
// when a schedule tile edge is 64 or the larger units would leave CUs idle),
// each split into four quadrants, one per wave; since schedule tiles are powers
// of two from 64 to 512 and at least as large as a quadrant, every quadrant
// lies in exactly one schedule tile, and a unit's quadrant mask holds the
// quadrants whose tile computes that plane.
//
// Export (reference api_export.cpp:365-410 with per-tile bounds): each tile is
// reconstructed with its own selected prefix and bound, zero-output tiles
// export 0; records are grouped by prefix so each group is one launch of the
// kernel instantiated for that prefix.
#include <algorithm>

#include "handles.hpp"

namespace rns8x {
namespace {

constexpr uint32_t kUnitGroupRows = 4;  // tile rows walked together (neighbours share A / B panels in L2)
constexpr uint64_t kLargeUnitsMin = 256;  // large units only when every CU gets one

template <typename T>
rns8_status upload(const std::vector<T>& host, T** dev, hipStream_t stream) {
  *dev = nullptr;
  if (host.empty()) return RNS8_SUCCESS;
  const std::size_t bytes = sizeof(T) * host.size();
  if (hipMalloc(reinterpret_cast<void**>(dev), bytes) != hipSuccess) {
    *dev = nullptr;
    return RNS8_BACKEND_FAILURE;
  }
  if (hipMemcpyAsync(*dev, host.data(), bytes, hipMemcpyHostToDevice, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return RNS8_BACKEND_FAILURE;
  return RNS8_SUCCESS;
}

bool zero_output(const rns8_plan_tile_schedule_entry& e) { return (e.flags & RNS8_TILE_SCHEDULE_ZERO_OUTPUT) != 0; }

}  // namespace

rns8_status upload_tile_lists(rns8_plan& p, hipStream_t stream) {
  if (!per_tile_kind(p.desc.bound_kind)) return RNS8_SUCCESS;
  const int64_t m = p.desc.m, n = p.desc.n;
  const uint32_t tm = p.desc.tile_m, tn = p.desc.tile_n;
  if (m <= 0 || n <= 0 || m >= (int64_t{1} << 31) || n >= (int64_t{1} << 31)) return RNS8_UNSUPPORTED_BACKEND;
  if (p.schedule.bounds.size() != p.tile_count) return RNS8_INTERNAL_ERROR;
  std::vector<rns8_plan_tile_schedule_entry> entries(p.tile_count);
  plan_tile_entries(p, entries.data());

  // export records, grouped by selected prefix; zero-output tiles first
  const bool is_signed = p.desc.semantics == RNS8_BOUNDED_I64;
  const uint64_t two63 = uint64_t{1} << 63;
  std::vector<TileExport> records;
  records.reserve(entries.size());
  p.export_groups.clear();
  for (uint32_t key = 0; key <= kMaxPrefix; ++key) {
    const uint32_t first = static_cast<uint32_t>(records.size());
    for (std::size_t i = 0; i < entries.size(); ++i) {
      const auto& e = entries[i];
      if ((zero_output(e) ? 0u : e.selected_prefix) != key) continue;
      const uint64_t b = p.schedule.bounds[i];
      TileExport r{};
      r.row_off = static_cast<uint32_t>(e.row_offset);
      r.col_off = static_cast<uint32_t>(e.col_offset);
      r.rows = static_cast<uint32_t>(e.row_extent);
      r.cols = static_cast<uint32_t>(e.col_extent);
      // |v| <= bound within int64 (crt.cpp:113-119), v <= bound for uint64
      r.pos64 = is_signed ? std::min(b, two63 - 1) : b;
      r.neg64 = is_signed ? std::min(b, two63) : 0u;
      if (r.rows == 0 || r.cols == 0 || r.rows > tm || r.cols > tn || e.row_offset + e.row_extent > m ||
          e.col_offset + e.col_extent > n)
        return RNS8_INTERNAL_ERROR;
      records.push_back(r);
    }
    const uint32_t count = static_cast<uint32_t>(records.size()) - first;
    if (count) p.export_groups.push_back(rns8_plan::ExportGroup{key, first, count});
  }

  // GEMM lists: only when the schedule did not collapse to the plan prefix
  std::vector<uint32_t> units;
  std::vector<TileFill> fills;
  if (!p.schedule.entries.empty()) {
    const uint32_t planes = storage_prefix(p);
    if (planes > kMaxPrefix) return RNS8_UNSUPPORTED_BACKEND;
    auto build_units = [&](uint32_t edge) -> bool {
      units.clear();
      const uint32_t quad = edge / 2;
      const uint64_t tiles_m64 = (static_cast<uint64_t>(m) + edge - 1) / edge;
      const uint64_t tiles_n64 = (static_cast<uint64_t>(n) + edge - 1) / edge;
      if (tiles_m64 >= (1u << 24) || tiles_n64 >= (1u << 24)) return false;
      const uint32_t tiles_m = static_cast<uint32_t>(tiles_m64), tiles_n = static_cast<uint32_t>(tiles_n64);
      auto quad_tile = [&](uint32_t tr, uint32_t tc, uint32_t q) -> const rns8_plan_tile_schedule_entry* {
        const int64_t r0 = int64_t{tr} * edge + (q >> 1) * quad;
        const int64_t c0 = int64_t{tc} * edge + (q & 1u) * quad;
        if (r0 >= m || c0 >= n) return nullptr;
        return &entries[static_cast<std::size_t>((r0 / tm) * static_cast<int64_t>(p.tile_cols) + c0 / tn)];
      };
      for (uint32_t plane = 0; plane < planes; ++plane)
        for (uint32_t g0 = 0; g0 < tiles_m; g0 += kUnitGroupRows)
          for (uint32_t tc = 0; tc < tiles_n; ++tc)
            for (uint32_t tr = g0; tr < std::min(tiles_m, g0 + kUnitGroupRows); ++tr) {
              uint32_t mask = 0;
              for (uint32_t q = 0; q < 4; ++q) {
                const auto* e = quad_tile(tr, tc, q);
                if (e && !zero_output(*e) && plane < e->selected_prefix) mask |= 1u << q;
              }
              if (!mask) continue;
              units.push_back(plane << 24 | tr);
              units.push_back(mask << 24 | tc);
            }
      return units.size() / 2 <= 0x7FFFFFFFu;
    };
    // 256 x 256 units (128 x 128 quadrants) run ~1.4x faster per MFMA op than
    // 128 x 128 ones; they need schedule tiles of at least 128 and enough units
    p.unit_edge = 128;
    if (tm >= 128 && tn >= 128 && build_units(256) && units.size() / 2 >= kLargeUnitsMin) p.unit_edge = 256;
    if (p.unit_edge == 128 && !build_units(128)) return RNS8_UNSUPPORTED_BACKEND;
    for (const auto& e : entries)
      if (zero_output(e))
        fills.push_back(TileFill{static_cast<uint32_t>(e.row_offset), static_cast<uint32_t>(e.col_offset),
                                 static_cast<uint32_t>(e.row_extent), static_cast<uint32_t>(e.col_extent),
                                 e.selected_prefix});
    for (const auto& f : fills)
      if (f.planes == 0 || f.planes > planes || f.col_off % 16 != 0) return RNS8_INTERNAL_ERROR;
  }

  rns8_status st = upload(units, &p.units, stream);
  if (st == RNS8_SUCCESS) st = upload(fills, &p.zero_fills, stream);
  if (st == RNS8_SUCCESS) st = upload(records, &p.export_tiles, stream);
  if (st != RNS8_SUCCESS) {
    free_tile_lists(p);
    return st;
  }
  p.unit_count = static_cast<uint32_t>(units.size() / 2);
  p.zero_fill_count = static_cast<uint32_t>(fills.size());
  return RNS8_SUCCESS;
}

void free_tile_lists(rns8_plan& p) {
  free_device(p.units);
  free_device(p.zero_fills);
  free_device(p.export_tiles);
  p.units = nullptr;
  p.zero_fills = nullptr;
  p.export_tiles = nullptr;
  p.unit_count = 0;
  p.zero_fill_count = 0;
  p.export_groups.clear();
}

}  // namespace rns8x
