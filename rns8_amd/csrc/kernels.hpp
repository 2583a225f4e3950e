// Host-side launchers for the gfx950 kernels (defined in the .hip files).
//
// Every launcher checks that the shapes it receives match what its grid and
// index arithmetic assume (non-negative sizes, 16-byte padded pitches,
// prefix <= 20) and returns hipErrorInvalidValue otherwise, so no kernel is
// launched with a geometry that could index outside its buffers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "exact_axes.hpp"
#include "tables.hpp"

namespace rns8x {

// ---- pack: native operand -> centered int8 residue planes ------------------
enum class NativeKind : uint32_t { I64 = 0, U64 = 1 };

struct PackArgs {
  const void* src;  // device, rows x cols elements at row stride `ld`
  int64_t rows;
  int64_t cols;
  int64_t ld;       // elements
  int8_t* planes;   // device, `nplanes` planes
  int64_t plane_ld; // padded_ld(cols)
  int64_t plane_pitch;
  uint32_t nplanes;
  NativeKind kind;
};
hipError_t launch_pack_native(const PackArgs& args, const PlaneConsts& consts, hipStream_t stream);

// ---- exact-wide magnitude proofs (exact_axes.hip) ---------------------------
// Per-row and per-column summaries of a rows x cols native operand (row
// stride ld elements) into out_rows / out_cols, and its max |x| into
// words[0] (words[1..7] zero). row_part / col_part: scratch for
// native_partial_rows(rows, cols) and native_partial_cols(rows, cols)
// partials (one per axis and 64 x 64 tile).
hipError_t launch_native_axes(const void* src, int64_t rows, int64_t cols, int64_t ld, bool is_signed,
                              xa::AxisPartial* row_part, xa::AxisPartial* col_part, xa::AxisRecord* out_rows,
                              xa::AxisRecord* out_cols, uint64_t* words, hipStream_t stream);
inline int64_t native_partial_rows(int64_t rows, int64_t cols) { return rows * ((cols + 63) / 64); }
inline int64_t native_partial_cols(int64_t rows, int64_t cols) { return cols * ((rows + 63) / 64); }
// The carried summaries of C = A x B (m x n, inner k): per-row and
// per-column maxima and sums of the cell bounds from A's m row records and
// B's n column records (kinds: xa::AxisKind; a uniform side reads no
// records), and C's bound into out_words[0..3] (out_words[4..7] zero).
// a_words / b_words: the operands' bounds, 4 words each.
hipError_t launch_product_axes(const xa::AxisRecord* arows, uint32_t akind, const xa::AxisRecord* bcols,
                               uint32_t bkind, const uint64_t* a_words, const uint64_t* b_words, int64_t m,
                               int64_t n, uint64_t k, xa::AxisRecord* out_rows, xa::AxisRecord* out_cols,
                               uint64_t* out_words, hipStream_t stream);
// Copies m row records, n column records, a_words[0..3] into out_words[0..3]
// and b_words[0..3] into out_words[4..7].
hipError_t launch_proof_snapshot(const xa::AxisRecord* arows, const xa::AxisRecord* bcols, const uint64_t* a_words,
                                 const uint64_t* b_words, int64_t m, int64_t n, xa::AxisRecord* out_rows,
                                 xa::AxisRecord* out_cols, uint64_t* out_words, hipStream_t stream);

struct PackU8Args {
  const uint8_t* src;
  int64_t rows;
  int64_t cols;
  int64_t ld;
  int8_t* plane;
  int64_t plane_ld;
  uint32_t modulus;
};
hipError_t launch_pack_u8(const PackU8Args& args, hipStream_t stream);

// ---- plane GEMM: C_p = center(A_p x B_p mod m_p) ---------------------------
struct GemmArgs {
  const int8_t* a;  // [planes][m][lda]
  const int8_t* b;  // [planes][k][ldb]
  int8_t* c;        // [planes][m][ldc]
  int64_t m, n, k;
  int64_t lda, ldb, ldc;  // padded pitches (bytes, multiples of 16)
  int64_t pitch_a, pitch_b, pitch_c;
  uint32_t nplanes;
  // split-K: the workspace of centered int8 residues [slices][planes][m][ldc]
  // (each slice writes its own slot; no zeroing needed; 16-byte aligned, as
  // is c) and the number of K slices; slices == 1 disables it.
  int8_t* splitk_ws;
  uint32_t slices;
};
hipError_t launch_gemm(const GemmArgs& args, const PlaneConsts& consts, hipStream_t stream);

// Fused native-input GEMM (fused.hip): C's residue planes straight from
// int64/uint64 device operands, for outputs small enough that the product is
// split along K. `shape` comes from choose_fused_shape, which returns false
// where the fused path is not offered (its int8 workspace of partial residues,
// [slices][planes][m][ldc], would exceed its limit).
struct FusedShape {
  uint32_t slices;    // K slices, each a multiple of 32 (64 for the skinny form) and at most 65536 deep
  int64_t k_slice;
  uint64_t ws_bytes;
  // results at most 16 columns wide (fused_skinny.hip): the workspace starts
  // with B's transposed residue planes (bt_bytes), then the slices' slots
  uint32_t skinny;
  uint64_t bt_bytes;
};
bool choose_fused_shape(int64_t m, int64_t n, int64_t k, uint32_t nplanes, int64_t ldc, FusedShape& out);
bool fused_skinny_shape(int64_t m, int64_t n, int64_t k, uint32_t nplanes, FusedShape& out);
// The fused path's operand requirements: a 16-byte aligned A with an even row
// stride below 2^21 elements; B likewise for the tile form, any 8-byte aligned
// B for the skinny form (its loads are scalar).
bool fused_operands_ok(const void* a, int64_t lda, const void* b, int64_t ldb, bool skinny);
struct FusedArgs {
  const void* a;  // device, m x k native elements at row stride lda
  const void* b;  // device, k x n native elements at row stride ldb
  int64_t lda, ldb;
  int64_t m, n, k;
  int8_t* c;  // [nplanes][m][ldc] centered residues
  int64_t ldc, pitch_c;
  uint32_t nplanes;
  NativeKind kind;
  int8_t* ws;  // shape.ws_bytes of workspace
  FusedShape shape;
};
// Whether launch_fused_native accepts `args` (it returns hipErrorInvalidValue
// otherwise, before enqueuing anything).
bool fused_args_ok(const FusedArgs& args);
hipError_t launch_fused_native(const FusedArgs& args, const PlaneConsts& consts, hipStream_t stream);
// The skinny form (shape.skinny), called by launch_fused_native once the
// arguments are checked.
hipError_t launch_fused_skinny(const FusedArgs& args, const PlaneConsts& consts, hipStream_t stream);
// Per-tile schedules: `units` edge x edge tile-planes (edge 256 or 128) from a
// device list of two words each, (plane << 24 | tile row) and (quadrant mask
// << 24 | tile column); bit q = 2 * (row half) + (column half) of the mask
// enables the stores of that edge/2 x edge/2 quadrant. No K split; K beyond
// 65536 runs as accumulating launches.
hipError_t launch_gemm_listed(const GemmArgs& args, const PlaneConsts& consts, const uint32_t* d_units,
                              uint32_t units, uint32_t edge, hipStream_t stream);
// Zero-output tiles: planes [0, planes) of each tile set to 0; records are
// checked against the shape where they are built.
struct TileFill {
  uint32_t row_off, col_off, rows, cols, planes;
};
hipError_t launch_zero_tiles(int8_t* c, int64_t ldc, int64_t pitch_c, const TileFill* d_tiles, uint32_t count,
                             hipStream_t stream);
// Grouped launches: tasks of one shape (the GemmArgs shape, pitches, planes
// and slices), each with its own operands, result and split-K workspace; one
// persistent launch per K block covers up to kMaxGroupTasks tasks, larger
// groups run as consecutive launches (reference api_gemm.cpp:1199-1210).
struct TaskPtrs {
  const int8_t* a;
  const int8_t* b;
  int8_t* c;
  int8_t* ws;  // split-K residues of this task (slices > 1 only)
};
constexpr uint32_t kMaxGroupTasks = 32;
hipError_t launch_gemm_grouped(const GemmArgs& shape, const PlaneConsts& consts, const TaskPtrs* tasks,
                               uint32_t count, hipStream_t stream);
// How launch_gemm runs a shape: the kernel (plane_gemm_kernel with 256 or
// 128 tiles, or the skinny kernel for results at most 16 columns wide) and
// the K split. A split covers the whole K in slices of at most 65536, each
// writing its centered residues to the int8 workspace, and a finalize adds
// them; unsplit products with K beyond 65536 run as accumulating launches.
struct GemmShape {
  int tile;           // 256, 128, or 16 (skinny kernel)
  uint32_t slices;    // K slices (1 = no split)
  int64_t k_slice;    // K of one slice
  uint64_t ws_bytes;  // workspace: slices * nplanes * m * padded_ld(n) bytes when split, else 0
};
GemmShape choose_gemm_shape(int64_t m, int64_t n, int64_t k, uint32_t nplanes);
// The skinny kernel's shape for n <= 16 (false for wider results), and its
// launcher (skinny.hip): B and C rows of 16 bytes, args.slices ==
// shape.slices.
bool skinny_shape(int64_t m, int64_t n, int64_t k, uint32_t nplanes, GemmShape& out);
hipError_t launch_skinny(const GemmArgs& args, const GemmShape& shape, const PlaneConsts& consts, hipStream_t stream);
// Adds the centered residues of `slices` workspace slots [slices][nplanes][m]
// [ldc] and writes their centered residue to C's planes (fused.hip). ws and c
// 16-byte aligned, ldc and pitch_c multiples of 16.
hipError_t launch_residue_finalize(const int8_t* ws, int8_t* c, int64_t m, int64_t ldc, int64_t pitch_c,
                                   uint32_t nplanes, uint32_t slices, const PlaneConsts& consts, hipStream_t stream);

// Per-device static split-K scratch (gemm.hip) for GEMM calls that bring no
// workspace and may allocate nothing: kNoAllocScratchBytes of int8 residues.
constexpr uint64_t kNoAllocScratchBytes = uint64_t{4} << 20;
// Records `device`'s address of the scratch (hipGetSymbolAddress), once per
// device; `device` must be the current device. Returns the HIP error of the
// lookup, or hipSuccess when the address is (already) recorded.
hipError_t resolve_noalloc_scratch(int device);
// The recorded address for `device`, or nullptr when it was never resolved.
int8_t* noalloc_scratch(int device);

// ---- export ------------------------------------------------------------------
enum class ExportKind : uint32_t { I64 = 0, U64 = 1, WIDE_SIGNED = 2, WIDE_UNSIGNED = 3 };

struct ExportArgs {
  const int8_t* c;  // [prefix][m][ldc] residue planes
  int64_t m, n;
  int64_t ldc;
  int64_t pitch_c;
  void* dst;        // device, element (r, col) at dst[(r*ld + col) * limbs]
  int64_t ld;       // elements
  uint32_t limbs;   // 64-bit limbs per element (1 for i64/u64)
  ExportKind kind;
  uint64_t bound;   // bounded kinds
  uint32_t* status; // device word; set nonzero on any range violation
};
hipError_t launch_export(const ExportArgs& args, uint32_t prefix, hipStream_t stream);

// Per-tile export (bounded int64 / uint64): one record per schedule tile,
// cells [row_off, row_off + rows) x [col_off, col_off + cols), admissible
// magnitudes pos64 (v >= 0) and neg64 (v < 0). The tiles of one call share
// the prefix; tile_m / tile_n are the schedule's tile edges (64 .. 512), which
// every record's extent is within. The records are checked against the shape
// where they are built.
struct TileExport {
  uint32_t row_off, col_off, rows, cols;
  uint64_t pos64, neg64;
};
hipError_t launch_export_tiles(const ExportArgs& a, uint32_t prefix, const TileExport* d_tiles, uint32_t count,
                               uint32_t tile_m, uint32_t tile_n, hipStream_t stream);
// Zero-output tiles: their cells of dst set to 0 (a.status is not used).
hipError_t launch_export_zero_tiles(const ExportArgs& a, const TileExport* d_tiles, uint32_t count, uint32_t tile_m,
                                    uint32_t tile_n, hipStream_t stream);

struct ExportU8Args {
  const int8_t* c;
  int64_t m, n;
  int64_t ldc;
  uint8_t* dst;
  int64_t ld;
  uint32_t modulus;
};
hipError_t launch_export_u8(const ExportU8Args& args, hipStream_t stream);

// The launchers' argument checks (contract.cpp): launch_gemm,
// launch_export, launch_export_u8, launch_pack_native and launch_pack_u8
// refuse (hipErrorInvalidValue) arguments these reject.
bool gemm_args_ok(const GemmArgs& a);
bool export_args_ok(const ExportArgs& a, uint32_t prefix);
bool export_u8_args_ok(const ExportU8Args& a);
bool pack_args_ok(const PackArgs& a);
bool pack_u8_args_ok(const PackU8Args& a);

// Fill `words` 32-bit words with zero (used instead of hipMemsetAsync so the
// call sequence stays valid under stream capture).
hipError_t launch_zero_words(uint32_t* dst, uint64_t words, hipStream_t stream);

}  // namespace rns8x
