/* rns8 CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference library's CPU_REFERENCE arithmetic
 * (pack -> per-modulus int32 ring GEMM with 65536-wide K blocks -> Garner/CRT
 * export). Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only as the checker or the timed CPU baseline; the
 * product library (rns8_amd/librns8.so) never links or calls it.
 *
 * Multiprecision (Boost cpp_int in the reference) is replaced by fixed
 * 256-bit unsigned limb arithmetic, which covers every value the path can
 * produce (modulus products < 2^155, exact-wide GEMM sums < 2^160).
 *
 * Every function cites the reference file:line it restates. Parity pins are
 * listed in the tests (tests/test_oracle_*.py); no oracle function is
 * unpinned.
 */
#ifndef RNS8_ORACLE_H
#define RNS8_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status values match rns8_status */
enum {
  ORC_SUCCESS = 0,
  ORC_INVALID_ARGUMENT = 1,
  ORC_UNSUPPORTED_BACKEND = 4,
  ORC_RANGE_ERROR = 5
};

/* ---- ladder and prefix selection ---------------------------------------- */
uint16_t orc_modulus(uint32_t index);                       /* internal.hpp:328-330 */
double orc_prefix_range_bits(uint32_t prefix);              /* moduli.cpp:21-30 */
int orc_ladder_pairwise_coprime(void);                      /* moduli.cpp:143-152 */
void orc_modulus_product(uint32_t prefix, uint64_t out[4]); /* moduli.cpp:164-170 */
uint32_t orc_required_prefix_for_range(const uint64_t range[4]); /* moduli.cpp:181-190 */
/* Plan prefix selection for the global (non per-tile) bound contracts:
 * validate_gemm_desc (moduli.cpp:295-387) + configure_plan_schedule global
 * branch (api_plan_schedule.inc:263-278) + schedule_required_range
 * (api_oneshot.cpp:473-502). Returns a status; *prefix_out on success. */
int orc_select_prefix(uint32_t semantics, uint32_t bound_kind, uint64_t bound, int64_t k, uint32_t max_prefix,
                      uint32_t flags, uint64_t lhs_bound, uint64_t rhs_bound, uint32_t* prefix_out);

/* ---- residues ------------------------------------------------------------ */
int8_t orc_centered_i64(int64_t value, uint32_t modulus);   /* cpu_reference.cpp:10-32 */
int8_t orc_centered_u64(uint64_t value, uint32_t modulus);  /* cpu_reference.cpp:10-32 */
int8_t orc_reduce_to_centered(int64_t value, uint32_t modulus); /* cpu_reference.cpp:34-44 */
uint32_t orc_canonical_from_centered(int8_t residue, uint32_t modulus); /* cpu_reference.cpp:18-24 */

/* planes are compact [prefix][rows][cols] (cpu_reference.cpp:46-51) */
void orc_pack_i64(const int64_t* src, int64_t rows, int64_t cols, int64_t ld, uint32_t prefix, int8_t* planes);
void orc_pack_u64(const uint64_t* src, int64_t rows, int64_t cols, int64_t ld, uint32_t prefix, int8_t* planes);
void orc_pack_finite_u8(const uint8_t* src, int64_t rows, int64_t cols, int64_t ld, uint32_t modulus,
                        int8_t* plane);

/* ---- ring GEMM ----------------------------------------------------------- */
/* cpu_reference.cpp:156-206 (one modulus, int32 blocks of 65536, centered) */
void orc_ring_gemm_modulus(const int8_t* A, const int8_t* B, int8_t* C, int64_t m, int64_t n, int64_t k,
                           int64_t lda, int64_t ldb, int64_t ldc, uint32_t modulus);
/* cpu_reference.cpp:221-284 non-tiled branch: planes 0..prefix-1 */
void orc_gemm_rns(const int8_t* A, const int8_t* B, int8_t* C, int64_t m, int64_t n, int64_t k,
                  uint32_t prefix);
/* residue_dot.hpp:21-38 (single cell, b at stride b_stride) */
int8_t orc_centered_residue_dot(const int8_t* a, const int8_t* b, int64_t k, int64_t b_stride,
                                uint32_t modulus);

/* ---- CRT / export -------------------------------------------------------- */
/* crt.cpp:54-76: canonical x in [0, P) as 4 little-endian u64 limbs */
void orc_reconstruct_canonical(const int8_t* residues, uint32_t prefix, uint64_t out[4]);
int orc_reconstruct_signed(const int8_t* residues, uint32_t prefix, uint64_t bound, int64_t* out);   /* crt.cpp:100-121 */
int orc_reconstruct_unsigned(const int8_t* residues, uint32_t prefix, uint64_t bound, uint64_t* out); /* crt.cpp:78-98 */
int orc_exact_wide_signed_limbs(const int8_t* residues, uint32_t prefix, uint64_t* out, uint32_t limbs);   /* crt.cpp:144-170 */
int orc_exact_wide_unsigned_limbs(const int8_t* residues, uint32_t prefix, uint64_t* out, uint32_t limbs); /* crt.cpp:123-142 */

/* Matrix exports over compact planes; staged, dst untouched unless every cell
 * succeeds; the status of the first failing cell (row-major) is returned
 * (api_export.cpp:365-414 and 631-716). */
int orc_export_i64(const int8_t* C, int64_t m, int64_t n, uint32_t prefix, uint64_t bound, int64_t* dst, int64_t ld);
int orc_export_u64(const int8_t* C, int64_t m, int64_t n, uint32_t prefix, uint64_t bound, uint64_t* dst, int64_t ld);
int orc_export_exact_wide_signed(const int8_t* C, int64_t m, int64_t n, uint32_t prefix, uint64_t* dst, int64_t ld,
                                 uint32_t limbs);
int orc_export_exact_wide_unsigned(const int8_t* C, int64_t m, int64_t n, uint32_t prefix, uint64_t* dst,
                                   int64_t ld, uint32_t limbs);
void orc_export_finite_u8(const int8_t* C, int64_t m, int64_t n, uint32_t modulus, uint8_t* dst, int64_t ld); /* cpu_reference.cpp:132-153 */

/* ---- per-tile bounded schedules ------------------------------------------- */
/* One tile of the schedule as rns8_get_plan_tile_schedule reports it
 * (rns8.h rns8_plan_tile_schedule_entry without the size/version header). */
typedef struct orc_tile_entry {
  uint32_t flags;
  uint64_t tile_row, tile_col;
  int64_t row_offset, col_offset, row_extent, col_extent;
  uint32_t required_prefix, selected_prefix, group_index, range_bit_length;
} orc_tile_entry;

typedef struct orc_schedule_summary {
  uint64_t tile_rows, tile_cols, tile_count;
  uint32_t min_required, max_required, min_selected, max_selected;
  uint32_t group_count, adaptive_prefix, adaptive_skip, range_bits, flags;
  uint64_t zero_a_row_count, zero_b_col_count, zero_row_col_product_count;
  uint32_t collapsed; /* 1: every tile runs the plan prefix; execution is the global one */
} orc_schedule_summary;

/* api_plan_schedule.inc:109-261 (per-tile branch) and
 * api_plan_public_api.inc:119-160 (entries reported for a collapsed schedule).
 * semantics: BOUNDED_I64 or BOUNDED_U64; budget = the plan prefix. */
int orc_tile_schedule(uint32_t semantics, int64_t m, int64_t n, uint32_t tile_m, uint32_t tile_n,
                      const uint64_t* tile_bounds, uint64_t count, uint32_t budget, uint32_t flags,
                      const uint8_t* zero_a_rows, const uint8_t* zero_b_cols, orc_tile_entry* entries,
                      orc_schedule_summary* summary);
/* cpu_reference.cpp:231-257: planes p < selected prefix of each tile; zero-output
 * tiles filled with 0; other planes of C left as they are. Compact planes. */
void orc_gemm_rns_tiled(const int8_t* A, const int8_t* B, int8_t* C, int64_t m, int64_t n, int64_t k,
                        const orc_tile_entry* entries, uint64_t count);
/* api_export.cpp:365-410: per cell the tile's selected prefix and bound; 0 for
 * zero-output tiles; dst untouched on the first failing status. C holds
 * `storage` compact planes. */
int orc_export_i64_tiled(const int8_t* C, int64_t m, int64_t n, uint32_t storage, uint32_t tile_m, uint32_t tile_n,
                         const orc_tile_entry* entries, const uint64_t* tile_bounds, uint64_t count, int64_t* dst,
                         int64_t ld);
int orc_export_u64_tiled(const int8_t* C, int64_t m, int64_t n, uint32_t storage, uint32_t tile_m, uint32_t tile_n,
                         const orc_tile_entry* entries, const uint64_t* tile_bounds, uint64_t count, uint64_t* dst,
                         int64_t ld);

/* ---- end-to-end CPU_REFERENCE path (api_oneshot.cpp:510-547, CS5) ------- */
/* pack -> gemm_rns -> export at an explicit prefix; rows [row0, row0+rows)
 * of C only (a bounded sample of a large GEMM uses row0/rows). */
int orc_gemm_i64_rows(const int64_t* A, int64_t lda, const int64_t* B, int64_t ldb, int64_t k, int64_t n,
                      int64_t row0, int64_t rows, uint32_t prefix, uint64_t bound, int64_t* C, int64_t ldc);
int orc_gemm_u64_rows(const uint64_t* A, int64_t lda, const uint64_t* B, int64_t ldb, int64_t k, int64_t n,
                      int64_t row0, int64_t rows, uint32_t prefix, uint64_t bound, uint64_t* C, int64_t ldc);
void orc_gemm_finite_u8_rows(const uint8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, int64_t k, int64_t n,
                             int64_t row0, int64_t rows, uint32_t modulus, uint8_t* C, int64_t ldc);
int orc_gemm_exact_wide_signed_rows(const int64_t* A, int64_t lda, const int64_t* B, int64_t ldb, int64_t k,
                                    int64_t n, int64_t row0, int64_t rows, uint32_t prefix, uint64_t* C,
                                    int64_t ldc, uint32_t limbs);

/* ---- brute-force exact GEMM (independent of RNS; cpu_reference.cpp:313-341) */
/* 256-bit two's complement sums, written as `limbs` little-endian u64 limbs */
void orc_exact_gemm_i64(const int64_t* A, int64_t lda, const int64_t* B, int64_t ldb, int64_t m, int64_t n,
                        int64_t k, uint64_t* C, int64_t ldc, uint32_t limbs);
void orc_exact_gemm_u64(const uint64_t* A, int64_t lda, const uint64_t* B, int64_t ldb, int64_t m, int64_t n,
                        int64_t k, uint64_t* C, int64_t ldc, uint32_t limbs);

/* ---- seeded inputs and checksum ----------------------------------------- */
/* SplitMix64 (Steele, Lea, Flood 2014) streams: state = seed; each draw adds
 * the golden gamma and mixes. */
uint64_t orc_splitmix64_next(uint64_t* state);
/* mode 0: int64 uniform in [-2^bits, 2^bits) via (x >> (63-bits)) - 2^bits
 * mode 1: uint64 uniform in [0, 2^bits) via x >> (64-bits)
 * mode 2: full 64-bit (x)
 * mode 3: byte uniform in [0, limit) by rejection of (x & 0xff) >= limit
 * Fills `count` 64-bit slots (modes 0-2) or bytes (mode 3). */
void orc_fill(uint64_t seed, uint32_t mode, uint32_t bits_or_limit, void* out, int64_t count);
/* FNV-1a style 64-bit mix over row-major values (rns8_bench_support.cpp:96-99) */
uint64_t orc_checksum_u64(const uint64_t* values, int64_t rows, int64_t cols, int64_t ld, uint32_t limbs);
uint64_t orc_checksum_u8(const uint8_t* values, int64_t rows, int64_t cols, int64_t ld);

int orc_num_threads(void);
void orc_set_num_threads(int threads);

#ifdef __cplusplus
}
#endif

#endif
