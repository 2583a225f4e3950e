// libFuzzer target over the pack -> GEMM -> export contract (contract.hpp),
// built with AddressSanitizer and UndefinedBehaviorSanitizer
// (tests/fuzz/Makefile). After the reference's
// tests/fuzz/rns8_fuzz_export_contract.cpp, which runs pack, rns8_gemm_rns and
// the exports (ld = n and n - 1) on its CPU backend for fuzzed shapes and
// values. This library has no CPU backend, so the target drives the host-side
// contract the ABI calls run before any kernel: the same validation
// functions, the kernel arguments a validated call builds, and the launchers'
// own checks of them, on host-only handles (planes at fixed fake addresses,
// never dereferenced).
//
// The input decodes into a plan descriptor of any storage semantics (global
// or per-tile bounds, dimensions from 1 to beyond the kernels' 32-bit
// limits), operand and result matrices derived from the plan and then, at
// random, perturbed (rows, columns, semantics, bound kind, prefix, tile grid,
// flags, currency, device, aliasing), a workspace, and pack sources and
// export destinations with fuzzed row strides and limb counts. Checked on
// every input, beyond the sanitizers:
//   * every check returns a status it is documented to return;
//   * matrices made for the plan, current and not aliased, are accepted, and
//     every perturbation that changes what the kernels would read is refused
//     with RNS8_INVALID_ARGUMENT (a stride below the row width included);
//   * an accepted GEMM, export or pack hands its launcher arguments the
//     launcher accepts, unless they exceed a documented kernel limit (32-bit
//     offsets and unit counts), and every plane, workspace and destination
//     byte the kernel can reach lies inside the matrix storage, the
//     workspace, or the caller's rows x ld x limbs elements.
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <vector>

#include "contract.hpp"

using namespace rns8x;

namespace {

struct Reader {
  const uint8_t* p;
  const uint8_t* end;
  uint64_t u64() {
    uint64_t v = 0;
    for (int i = 0; i < 8 && p < end; ++i) v |= static_cast<uint64_t>(*p++) << (8 * i);
    return v;
  }
  uint8_t u8() { return p < end ? *p++ : 0; }
};

void fail(const char* what, long long a = 0, long long b = 0) {
  std::fprintf(stderr, "FUZZ CHECK FAILED: %s (%lld, %lld)\n", what, a, b);
  std::abort();
}

// a dimension: mostly small, sometimes near the kernels' 32-bit limits
int64_t dim(Reader& r) {
  const uint8_t sel = r.u8();
  const uint64_t v = r.u64();
  switch (sel % 8) {
    case 0: return static_cast<int64_t>(v % (uint64_t{1} << 34)) + 1;
    case 1: return (int64_t{1} << (23 + v % 10)) - 1 + static_cast<int64_t>((v >> 8) % 3);
    case 2: return static_cast<int64_t>(v % 70000) + 1;
    default: return static_cast<int64_t>(v % 300) + 1;
  }
}

// a row stride for a rows x cols operand: at, below or above cols, or huge
int64_t stride(Reader& r, int64_t cols) {
  const uint8_t sel = r.u8();
  const uint64_t v = r.u64();
  switch (sel % 8) {
    case 0: return cols - 1;
    case 1: return cols + static_cast<int64_t>(v % 1000);
    case 2: return static_cast<int64_t>(v >> 1);
    case 3: return -static_cast<int64_t>(v % 5);
    default: return cols;
  }
}

const rns8_semantics kSem[] = {RNS8_BOUNDED_I64,        RNS8_BOUNDED_U64, RNS8_EXACT_WIDE_SIGNED,
                               RNS8_EXACT_WIDE_UNSIGNED, RNS8_FINITE_FIELD_U8, RNS8_FINITE_RING_U8};

// Fake, 256-byte aligned plane and buffer addresses, far apart (never used).
int8_t* fake(uint64_t i) { return reinterpret_cast<int8_t*>((i + 1) << 44); }

// The fields a perturbation may change, and whether the change alters what
// the kernels would read (must be refused) or not (must be accepted).
enum class Perturb { None, Rows, Cols, Semantics, BoundKind, SmallerPrefix, Flags, Layout, LargerPrefix, Tiles };

bool breaking(Perturb p, bool per_tile_plan) {
  switch (p) {
    case Perturb::None:
    case Perturb::LargerPrefix:
      return false;
    case Perturb::Tiles:
      return per_tile_plan;  // the tile grid is part of a per-tile matrix's contract only
    default:
      return true;
  }
}

struct Operand {
  rns8_matrix m;
  bool ok = false;  // init_matrix succeeded
  Perturb perturb = Perturb::None;
};

void make_operand(Reader& r, const rns8_plan& plan, int64_t rows, int64_t cols, uint64_t index, Operand& op) {
  const bool finite = uses_finite_storage(plan.desc.semantics);
  rns8_matrix_desc d{};
  d.struct_size = sizeof(d);
  d.abi_version = RNS8_ABI_VERSION;
  d.rows = rows;
  d.cols = cols;
  d.logical_ld = cols;
  d.semantics = plan.desc.semantics;
  d.logical_layout = RNS8_LAYOUT_ROW_MAJOR;
  d.bound_kind = finite ? RNS8_BOUND_NONE : storage_bound_kind(plan);
  d.max_prefix = finite ? 0 : storage_prefix(plan);
  d.tile_m = plan.desc.tile_m;
  d.tile_n = plan.desc.tile_n;
  const uint8_t sel = r.u8();
  if (sel % 3 == 0) {
    switch ((sel / 3) % 9) {
      case 0: d.rows += (sel & 0x80) ? 1 : -1; op.perturb = Perturb::Rows; break;
      case 1: d.cols += (sel & 0x80) ? 1 : -1; op.perturb = Perturb::Cols; break;
      case 2: {
        int idx = 0;
        while (kSem[idx] != plan.desc.semantics) ++idx;
        d.semantics = kSem[(idx + 1 + r.u8() % 5) % 6];  // any other storage semantics
        op.perturb = Perturb::Semantics;
        break;
      }
      case 3: d.bound_kind = static_cast<rns8_bound_kind>((d.bound_kind + 1 + r.u8() % 5) % 7); op.perturb = Perturb::BoundKind; break;
      case 4:
        if (!finite && d.max_prefix > 1) {
          d.max_prefix -= 1;
          op.perturb = Perturb::SmallerPrefix;
        }
        break;
      case 5: d.flags = 1u << (r.u8() % 32); op.perturb = Perturb::Flags; break;
      case 6: d.logical_layout = static_cast<rns8_layout>(2 + r.u8() % 2); op.perturb = Perturb::Layout; break;
      case 7:
        if (!finite && d.max_prefix < 20) {
          d.max_prefix += 1;
          op.perturb = Perturb::LargerPrefix;
        }
        break;
      default:
        d.tile_m = d.tile_m == 64 ? 128 : 64;
        op.perturb = Perturb::Tiles;
        break;
    }
  }
  const rns8_status st = init_matrix(d, RNS8_BACKEND_HIP_DIRECT, 0, op.m);
  if (st != RNS8_SUCCESS && st != RNS8_INVALID_ARGUMENT && st != RNS8_RANGE_ERROR && st != RNS8_UNSUPPORTED_BACKEND)
    fail("init_matrix status", st);
  op.ok = st == RNS8_SUCCESS;
  if (!op.ok) return;
  if (op.m.plane_bytes != static_cast<uint64_t>(op.m.plane_pitch) * op.m.prefix || op.m.plane_pitch < rows)
    fail("matrix layout");
  op.m.planes = fake(index);
  op.m.device_current = true;
  op.m.finite_modulus = static_cast<uint16_t>(plan.desc.finite_modulus);
}

// bytes [0, reach) of the planes a kernel can touch: planes [0, planes) of
// rows x ld bytes each
void check_plane_reach(const rns8_matrix& m, uint32_t planes, int64_t rows, int64_t ld, int64_t pitch,
                       const char* what) {
  if (planes == 0 || planes > m.prefix || pitch != m.plane_pitch || ld != m.plane_ld) fail(what, planes, m.prefix);
  if (rows > m.desc.rows || ld <= 0 || rows > std::numeric_limits<int64_t>::max() / ld) fail(what, rows);
  const uint64_t reach = static_cast<uint64_t>(planes - 1) * static_cast<uint64_t>(pitch) +
                         static_cast<uint64_t>(rows) * static_cast<uint64_t>(ld);
  if (static_cast<uint64_t>(rows) * static_cast<uint64_t>(ld) > static_cast<uint64_t>(pitch) || reach > m.plane_bytes)
    fail(what, static_cast<long long>(reach), static_cast<long long>(m.plane_bytes));
}

}  // namespace

extern "C" int LLVMFuzzerTestOneInput(const uint8_t* data, std::size_t size) {
  Reader r{data, data + size};
  rns8_gemm_desc d;
  std::memset(&d, 0, sizeof(d));
  d.struct_size = sizeof(d);
  d.abi_version = RNS8_ABI_VERSION;
  const uint8_t head = r.u8();
  d.semantics = kSem[head % 6];
  const bool finite = uses_finite_storage(d.semantics);
  d.m = dim(r);
  d.n = dim(r);
  d.k = dim(r);
  d.max_prefix = r.u8() % 21;
  d.flags = (head & 0x40) ? RNS8_PLAN_FORCE_FIXED_PREFIX : 0u;
  static const uint32_t kTiles[] = {64, 128, 256, 512};
  d.tile_m = kTiles[r.u8() % 4];
  d.tile_n = kTiles[r.u8() % 4];
  std::vector<uint64_t> bounds;
  if (finite) {
    static const uint16_t kPrimes[] = {2, 3, 7, 251, 127, 13};
    d.finite_modulus = d.semantics == RNS8_FINITE_FIELD_U8 ? kPrimes[r.u8() % 6] : static_cast<uint16_t>(2 + r.u8() % 255);
    d.bound_kind = RNS8_BOUND_NONE;
  } else if (exact_wide(d.semantics)) {
    d.bound_kind = RNS8_BOUND_NONE;
  } else {
    const bool sgn = d.semantics == RNS8_BOUNDED_I64;
    const uint64_t tiles = static_cast<uint64_t>((d.m + d.tile_m - 1) / d.tile_m) * ((d.n + d.tile_n - 1) / d.tile_n);
    if ((head & 0x80) && tiles <= 64) {
      d.bound_kind = sgn ? RNS8_BOUND_PER_TILE_MAX_ABS : RNS8_BOUND_PER_TILE_MAX_UNSIGNED;
      bounds.resize(tiles);
      for (auto& b : bounds) b = r.u8() % 4 == 0 ? r.u64() >> (r.u8() % 64) : r.u8();
      if (sgn)
        for (auto& b : bounds) b = b > (uint64_t{1} << 63) ? (uint64_t{1} << 63) : b;
      d.tile_bounds = bounds.data();
      d.tile_bounds_count = bounds.size();
    } else {
      d.bound_kind = sgn ? RNS8_BOUND_GLOBAL_MAX_ABS : RNS8_BOUND_GLOBAL_MAX_UNSIGNED;
      d.bound = r.u8() % 2 ? r.u64() >> (r.u8() % 64) : r.u64() % 5000;
      if (sgn && d.bound > (uint64_t{1} << 63)) d.bound = uint64_t{1} << 63;
    }
  }
  rns8_plan plan;
  const rns8_status ps = init_plan(d, RNS8_BACKEND_HIP_DIRECT, plan);
  if (ps != RNS8_SUCCESS && ps != RNS8_INVALID_ARGUMENT && ps != RNS8_RANGE_ERROR && ps != RNS8_UNSUPPORTED_BACKEND)
    fail("init_plan status", ps);
  if (ps != RNS8_SUCCESS) return 0;
  plan.device_id = 0;
  const bool per_tile_plan = per_tile_kind(plan.desc.bound_kind);
  const bool listed = per_tile_plan && !plan.schedule.entries.empty();

  rns8_context ctx;
  ctx.backend = RNS8_BACKEND_HIP_DIRECT;
  ctx.device_id = 0;

  Operand A, B, C;
  make_operand(r, plan, plan.desc.m, plan.desc.k, 0, A);
  make_operand(r, plan, plan.desc.k, plan.desc.n, 1, B);
  make_operand(r, plan, plan.desc.m, plan.desc.n, 2, C);

  // ---- GEMM ----------------------------------------------------------------
  rns8_workspace ws;
  ws.backend = plan.backend;
  ws.semantics = plan.desc.semantics;
  ws.bound_kind = plan.desc.bound_kind;
  ws.m = plan.desc.m;
  ws.n = plan.desc.n;
  ws.k = plan.desc.k;
  ws.prefix = plan.prefix;
  ws.finite_modulus = plan.desc.finite_modulus;
  ws.device_id = 0;
  ws.splitk_bytes = plan.splitk_bytes;
  ws.splitk = plan.splitk_bytes ? fake(3) : nullptr;
  const uint8_t gsel = r.u8();
  bool ws_short = false;
  if (gsel % 8 == 0 && ws.splitk_bytes > 0) {
    ws.splitk_bytes -= 1;
    ws_short = true;
  }
  const bool alias = gsel % 16 == 1;
  const bool a_stale = gsel % 16 == 2;
  if (A.ok && a_stale) A.m.device_current = false;
  if (A.ok && B.ok && C.ok) {
    const rns8_matrix& Cm = alias ? A.m : C.m;
    rns8_status st = check_plan_ctx_ws(ctx, plan, ws);
    if (st != RNS8_SUCCESS && st != RNS8_WORKSPACE_TOO_SMALL && st != RNS8_INVALID_ARGUMENT) fail("ws status", st);
    if ((st == RNS8_WORKSPACE_TOO_SMALL) != ws_short) fail("workspace check", st, ws_short);
    if (st == RNS8_SUCCESS)
      st = finite ? check_finite_operands(ctx, plan, static_cast<uint16_t>(plan.desc.finite_modulus), A.m, B.m, Cm)
                  : check_rns_operands(ctx, plan, A.m, B.m, Cm);
    if (st != RNS8_SUCCESS && st != RNS8_INVALID_ARGUMENT && st != RNS8_WORKSPACE_TOO_SMALL) fail("gemm status", st);
    const bool broken = breaking(A.perturb, per_tile_plan) || breaking(B.perturb, per_tile_plan) ||
                        breaking(C.perturb, per_tile_plan) || alias || a_stale;
    if (!ws_short && broken != (st != RNS8_SUCCESS))
      fail("gemm acceptance (status; perturbations of A, B, C)", st,
           static_cast<int>(A.perturb) * 100 + static_cast<int>(B.perturb) * 10 + static_cast<int>(C.perturb));
    if (st == RNS8_SUCCESS) {
      const uint32_t nplanes = finite ? 1u : listed ? storage_prefix(plan) : plan.prefix;
      const uint32_t slices = listed ? 1u : plan.splitk_slices;
      const GemmArgs g = gemm_args(plan, A.m, B.m, Cm, ws.splitk, nplanes, slices);
      if (gemm_args_ok(g)) {
        check_plane_reach(A.m, nplanes, g.m, g.lda, g.pitch_a, "A reach");
        check_plane_reach(B.m, nplanes, g.k, g.ldb, g.pitch_b, "B reach");
        check_plane_reach(Cm, nplanes, g.m, g.ldc, g.pitch_c, "C reach");
        if (g.lda < g.k || g.ldb < g.n || g.ldc < g.n) fail("GEMM strides");
        if (slices > 1) {
          // [slices][planes][m][ldc] residue slots
          const uint64_t need = static_cast<uint64_t>(slices) * nplanes * static_cast<uint64_t>(g.m) *
                                static_cast<uint64_t>(g.ldc);
          if (need > ws.splitk_bytes) fail("split-K workspace reach", static_cast<long long>(need));
        }
      } else if (!(g.lda >= (int64_t{1} << 23) || g.ldb >= (int64_t{1} << 23) || g.m >= (int64_t{1} << 31))) {
        fail("validated GEMM refused by its launcher", g.lda, g.ldb);
      }
    }
  }

  // ---- export ----------------------------------------------------------------
  if (C.ok) {
    const int64_t m = plan.desc.m, n = plan.desc.n;
    const int64_t ld = stride(r, n);
    const bool stale = r.u8() % 16 == 0;
    if (stale) C.m.device_current = false;
    rns8_status st;
    uint32_t limbs = 1;
    ExportKind kind = ExportKind::I64;
    if (finite) {
      st = valid_access(m, n, ld) ? check_finite_export(ctx, plan, static_cast<uint16_t>(plan.desc.finite_modulus), C.m)
                                  : RNS8_INVALID_ARGUMENT;
    } else {
      kind = plan.desc.semantics == RNS8_BOUNDED_I64   ? ExportKind::I64
             : plan.desc.semantics == RNS8_BOUNDED_U64 ? ExportKind::U64
             : plan.desc.semantics == RNS8_EXACT_WIDE_SIGNED ? ExportKind::WIDE_SIGNED
                                                             : ExportKind::WIDE_UNSIGNED;
      if (exact_wide(plan.desc.semantics)) limbs = r.u8() % 34;
      const bool access = exact_wide(plan.desc.semantics) ? valid_limb_access(m, n, ld, limbs) : valid_access(m, n, ld);
      st = access ? check_export(ctx, plan, C.m, plan.desc.semantics) : RNS8_INVALID_ARGUMENT;
    }
    if (st != RNS8_SUCCESS && st != RNS8_INVALID_ARGUMENT && st != RNS8_RANGE_ERROR) fail("export status", st);
    if (ld < n && st != RNS8_INVALID_ARGUMENT) fail("export accepted ld < n", ld, n);
    const bool broken = breaking(C.perturb, per_tile_plan) || stale;
    if (broken && st == RNS8_SUCCESS) fail("export of a mismatched matrix accepted");
    if (st == RNS8_SUCCESS) {
      // the caller's buffer: rows x ld elements of `limbs` 64-bit limbs (one byte for finite
      // results), counted in limbs: the entry points bound element counts, not byte counts
      const uint64_t elem = finite ? 1u : limbs;
      const uint64_t buffer = static_cast<uint64_t>(m) * static_cast<uint64_t>(ld) * elem;
      const uint64_t reach = (static_cast<uint64_t>(m - 1) * static_cast<uint64_t>(ld) + static_cast<uint64_t>(n)) * elem;
      if (reach > buffer) fail("destination reach");
      if (finite) {
        const ExportU8Args a = export_u8_args(plan, C.m, reinterpret_cast<uint8_t*>(fake(5)), ld,
                                              static_cast<uint16_t>(plan.desc.finite_modulus));
        if (export_u8_args_ok(a)) check_plane_reach(C.m, 1, m, a.ldc, C.m.plane_pitch, "finite export reach");
        else if (a.ldc / 16 <= 0xFFFFFFFFll) fail("validated finite export refused by its launcher");
      } else if (!per_tile_plan) {
        // device export into the caller's rows; host export into compact staging (ld = n)
        for (int64_t dld : {ld, n}) {
          const ExportArgs a = export_args(plan, C.m, fake(6), dld, limbs, kind, reinterpret_cast<uint32_t*>(fake(7)));
          if (export_args_ok(a, plan.prefix)) check_plane_reach(C.m, plan.prefix, m, a.ldc, a.pitch_c, "export reach");
          else if (a.ldc / 4 <= 0xFFFFFFFFll) fail("validated export refused by its launcher", dld, limbs);
        }
      }
    }
  }

  // ---- pack ------------------------------------------------------------------
  if (A.ok) {
    const int64_t ld = stride(r, A.m.desc.cols);
    const uint8_t psel = r.u8();
    rns8_status st;
    if (finite) {
      const uint16_t mod = psel % 4 == 0 ? static_cast<uint16_t>(r.u8() + r.u8()) : static_cast<uint16_t>(plan.desc.finite_modulus);
      st = check_pack_u8(ctx, A.m, mod, ld);
      if (st != RNS8_SUCCESS && st != RNS8_INVALID_ARGUMENT) fail("pack u8 status", st);
      if (st == RNS8_SUCCESS) {
        const PackU8Args a = pack_u8_args(A.m, reinterpret_cast<const uint8_t*>(fake(8)), ld, mod);
        if (pack_u8_args_ok(a))
          check_plane_reach(A.m, 1, A.m.desc.rows, a.plane_ld, A.m.plane_pitch, "pack u8 reach");
        else if (a.rows <= (int64_t{1} << 32) / (a.plane_ld / 16) && (a.plane_ld / 16) * a.rows < (int64_t{1} << 32))
          fail("validated finite pack refused by its launcher", A.m.desc.rows, a.plane_ld);
      }
    } else {
      const bool sgn = psel & 1;
      st = check_pack_native(ctx, A.m, ld, sgn);
      if (st != RNS8_SUCCESS && st != RNS8_INVALID_ARGUMENT) fail("pack status", st);
      const bool kind_ok = A.m.desc.semantics == (sgn ? RNS8_BOUNDED_I64 : RNS8_BOUNDED_U64) ||
                           A.m.desc.semantics == (sgn ? RNS8_EXACT_WIDE_SIGNED : RNS8_EXACT_WIDE_UNSIGNED);
      if (st == RNS8_SUCCESS && (!kind_ok || ld < A.m.desc.cols)) fail("pack accepted a wrong kind or ld < cols");
      if (st == RNS8_SUCCESS) {
        const PackArgs a = pack_args(A.m, fake(9), ld, sgn);
        if (pack_args_ok(a)) {
          check_plane_reach(A.m, A.m.prefix, A.m.desc.rows, a.plane_ld, a.plane_pitch, "pack reach");
        } else if ((a.plane_ld / 8) * a.rows < (int64_t{1} << 32)) {
          fail("validated pack refused by its launcher", a.rows, a.plane_ld);
        }
      }
    }
  }
  return 0;
}
