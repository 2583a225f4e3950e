/* rns8 CPU oracle -- TEST INFRASTRUCTURE ONLY (see rns8_oracle.h).
 *
 * Restates the reference CPU_REFERENCE path with native integers:
 *   src/cpu/cpu_reference.cpp      pack, ring GEMM, finite export
 *   src/reconstruct/crt.cpp        Garner reconstruct, bounded/limb export
 *   src/core/moduli.cpp            ladder, products, prefix selection
 *   src/core/api_export.cpp        staged matrix export (dst untouched on error)
 *   src/backend_common/residue_dot.hpp  K-blocked residue dot
 * cpp_int is replaced by 4-limb (256-bit) unsigned arithmetic.
 */
#include "rns8_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_MAX_PREFIX 20u
#define ORC_LADDER 28u
#define ORC_K_BLOCK 65536
#define SEM_BOUNDED_I64 1u
#define SEM_BOUNDED_U64 2u
#define SEM_EW_SIGNED 3u
#define SEM_EW_UNSIGNED 4u
#define SEM_FINITE_RING 6u
#define SEM_FINITE_FIELD 7u
#define BK_NONE 0u
#define BK_MAX_ABS 1u
#define BK_MAX_UNSIGNED 2u
#define BK_INPUT_RANGE 5u
#define FLAG_FORCE_FIXED 1u

/* src/core/internal.hpp:328-330 */
static const uint16_t kLadder[ORC_LADDER] = {256, 255, 253, 251, 247, 239, 233, 229, 227, 223,
                                              217, 211, 199, 197, 193, 191, 181, 179, 173, 167,
                                              163, 157, 151, 149, 139, 137, 131, 127};

/* ---- 256-bit unsigned helpers (little-endian limbs) --------------------- */

typedef struct { uint64_t w[4]; } u256;

static u256 u256_of(uint64_t v) { u256 r = {{v, 0, 0, 0}}; return r; }
static int u256_cmp(const u256* a, const u256* b) {
  for (int i = 3; i >= 0; --i) {
    if (a->w[i] != b->w[i]) return a->w[i] < b->w[i] ? -1 : 1;
  }
  return 0;
}
static u256 u256_add(u256 a, const u256* b) {
  unsigned __int128 c = 0;
  for (int i = 0; i < 4; ++i) {
    c += (unsigned __int128)a.w[i] + b->w[i];
    a.w[i] = (uint64_t)c;
    c >>= 64;
  }
  return a;
}
static u256 u256_sub(u256 a, const u256* b) {
  unsigned __int128 borrow = 0;
  for (int i = 0; i < 4; ++i) {
    unsigned __int128 d = (unsigned __int128)a.w[i] - b->w[i] - borrow;
    a.w[i] = (uint64_t)d;
    borrow = (d >> 64) ? 1 : 0;
  }
  return a;
}
static u256 u256_mul_u64(u256 a, uint64_t m) {
  unsigned __int128 c = 0;
  for (int i = 0; i < 4; ++i) {
    c += (unsigned __int128)a.w[i] * m;
    a.w[i] = (uint64_t)c;
    c >>= 64;
  }
  return a;
}
static uint32_t u256_mod_small(const u256* a, uint32_t m) {
  unsigned __int128 r = 0;
  for (int i = 3; i >= 0; --i) r = ((r << 64) | a->w[i]) % m;
  return (uint32_t)r;
}
static u256 u256_shl(u256 a, unsigned s) {
  while (s >= 64) { a.w[3] = a.w[2]; a.w[2] = a.w[1]; a.w[1] = a.w[0]; a.w[0] = 0; s -= 64; }
  if (s) {
    for (int i = 3; i > 0; --i) a.w[i] = (a.w[i] << s) | (a.w[i - 1] >> (64 - s));
    a.w[0] <<= s;
  }
  return a;
}
static u256 u256_pow2(unsigned bits) { return u256_shl(u256_of(1), bits); }

/* ---- ladder ------------------------------------------------------------- */

uint16_t orc_modulus(uint32_t index) { return index < ORC_LADDER ? kLadder[index] : 0; }

/* moduli.cpp:21-30 */
double orc_prefix_range_bits(uint32_t prefix) {
  if (prefix == 0 || prefix > ORC_LADDER) return 0.0;
  long double bits = 0.0L;
  for (uint32_t i = 0; i < prefix; ++i) bits += log2l((long double)kLadder[i]);
  return (double)bits;
}

static uint32_t gcd_u32(uint32_t a, uint32_t b) {
  while (b) { uint32_t t = a % b; a = b; b = t; }
  return a;
}

/* moduli.cpp:143-152 */
int orc_ladder_pairwise_coprime(void) {
  for (uint32_t i = 0; i < ORC_LADDER; ++i)
    for (uint32_t j = i + 1; j < ORC_LADDER; ++j)
      if (gcd_u32(kLadder[i], kLadder[j]) != 1) return 0;
  return 1;
}

static u256 modulus_product(uint32_t prefix) {
  u256 p = u256_of(1);
  for (uint32_t i = 0; i < prefix; ++i) p = u256_mul_u64(p, kLadder[i]);
  return p;
}

/* moduli.cpp:164-170 */
void orc_modulus_product(uint32_t prefix, uint64_t out[4]) {
  u256 p = modulus_product(prefix);
  memcpy(out, p.w, sizeof(p.w));
}

static uint32_t required_prefix(const u256* range) {
  u256 p = u256_of(1);
  for (uint32_t prefix = 1; prefix <= ORC_MAX_PREFIX; ++prefix) {
    p = u256_mul_u64(p, kLadder[prefix - 1]);
    if (u256_cmp(&p, range) > 0) return prefix;
  }
  return 0;
}

/* moduli.cpp:181-190 */
uint32_t orc_required_prefix_for_range(const uint64_t range[4]) {
  u256 r;
  memcpy(r.w, range, sizeof(r.w));
  return required_prefix(&r);
}

/* moduli.cpp:192-206 */
static uint32_t default_prefix(uint32_t semantics) {
  switch (semantics) {
    case SEM_BOUNDED_I64:
    case SEM_BOUNDED_U64: return 9;
    case SEM_EW_SIGNED:
    case SEM_EW_UNSIGNED: return 20;
    default: return 0;
  }
}

int orc_select_prefix(uint32_t semantics, uint32_t bound_kind, uint64_t bound, int64_t k, uint32_t max_prefix,
                      uint32_t flags, uint64_t lhs_bound, uint64_t rhs_bound, uint32_t* prefix_out) {
  const uint32_t budget = max_prefix ? max_prefix : default_prefix(semantics);
  if (k <= 0) return ORC_INVALID_ARGUMENT;
  if (semantics != SEM_BOUNDED_I64 && semantics != SEM_BOUNDED_U64 && semantics != SEM_EW_SIGNED &&
      semantics != SEM_EW_UNSIGNED)
    return ORC_UNSUPPORTED_BACKEND;
  u256 range;
  const u256 two63 = u256_pow2(63);
  if (semantics == SEM_EW_SIGNED || semantics == SEM_EW_UNSIGNED) {
    /* moduli.cpp:346-357, api_oneshot.cpp:494-497 */
    if (bound_kind != BK_NONE || bound != 0) return ORC_INVALID_ARGUMENT;
    if (budget == 0 || budget > ORC_MAX_PREFIX) return ORC_INVALID_ARGUMENT;
    range = u256_shl(u256_of((uint64_t)k), semantics == SEM_EW_SIGNED ? 127 : 128);
  } else if (bound_kind == BK_INPUT_RANGE) {
    /* moduli.cpp:208-232 then 366-383 */
    if (bound != 0) return ORC_INVALID_ARGUMENT;
    if (semantics == SEM_BOUNDED_I64 && (lhs_bound > (1ull << 63) || rhs_bound > (1ull << 63)))
      return ORC_RANGE_ERROR;
    u256 out = u256_mul_u64(u256_mul_u64(u256_of((uint64_t)k), lhs_bound), rhs_bound);
    const u256 limit = semantics == SEM_BOUNDED_I64 ? two63 : u256_of(UINT64_MAX);
    if (u256_cmp(&out, &limit) > 0) return ORC_RANGE_ERROR;
    range = semantics == SEM_BOUNDED_I64 ? u256_mul_u64(out, 2) : out;
  } else if (semantics == SEM_BOUNDED_I64) {
    /* moduli.cpp:246-266 */
    if (bound_kind != BK_MAX_ABS) return bound_kind == BK_MAX_UNSIGNED || bound_kind == BK_NONE
                                              ? ORC_INVALID_ARGUMENT
                                              : ORC_UNSUPPORTED_BACKEND;
    if (bound > (1ull << 63)) return ORC_INVALID_ARGUMENT;
    range = u256_mul_u64(u256_of(bound), 2);
  } else {
    /* moduli.cpp:267-283 */
    if (bound_kind != BK_MAX_UNSIGNED) return bound_kind == BK_MAX_ABS || bound_kind == BK_NONE
                                                   ? ORC_INVALID_ARGUMENT
                                                   : ORC_UNSUPPORTED_BACKEND;
    range = u256_of(bound);
  }
  if (budget == 0 || budget > ORC_MAX_PREFIX) return ORC_INVALID_ARGUMENT;
  const u256 product = modulus_product(budget);
  if (u256_cmp(&product, &range) <= 0) return ORC_RANGE_ERROR;
  /* api_plan_schedule.inc:263-278 */
  const uint32_t required = required_prefix(&range);
  if (required == 0 || required > budget) return ORC_RANGE_ERROR;
  *prefix_out = (flags & FLAG_FORCE_FIXED) ? budget : required;
  return ORC_SUCCESS;
}

/* ---- residues ------------------------------------------------------------ */

/* cpu_reference.cpp:10-32: canonical residue then centre at (m+1)/2 */
static int8_t center_canonical(uint32_t canonical, uint32_t modulus) {
  const uint32_t threshold = (modulus + 1u) / 2u;
  return (int8_t)(canonical >= threshold ? (int)canonical - (int)modulus : (int)canonical);
}

int8_t orc_centered_i64(int64_t value, uint32_t modulus) {
  __int128 r = (__int128)value % (__int128)modulus;
  if (r < 0) r += modulus;
  return center_canonical((uint32_t)r, modulus);
}

int8_t orc_centered_u64(uint64_t value, uint32_t modulus) {
  return center_canonical((uint32_t)(value % modulus), modulus);
}

/* cpu_reference.cpp:34-44 */
int8_t orc_reduce_to_centered(int64_t value, uint32_t modulus) {
  int64_t r = value % (int64_t)modulus;
  if (r < 0) r += modulus;
  const int64_t threshold = ((int64_t)modulus + 1) / 2;
  if (r >= threshold) r -= modulus;
  return (int8_t)r;
}

/* cpu_reference.cpp:18-24 */
uint32_t orc_canonical_from_centered(int8_t residue, uint32_t modulus) {
  const int v = residue;
  return v < 0 ? (uint32_t)(v + (int)modulus) : (uint32_t)v;
}

/* cpu_reference.cpp:53-79 (plane-row parallel) */
void orc_pack_i64(const int64_t* src, int64_t rows, int64_t cols, int64_t ld, uint32_t prefix, int8_t* planes) {
  const int64_t plane_rows = (int64_t)prefix * rows;
#pragma omp parallel for schedule(static)
  for (int64_t pr = 0; pr < plane_rows; ++pr) {
    const uint32_t p = (uint32_t)(pr / rows);
    const int64_t row = pr % rows;
    const uint32_t m = kLadder[p];
    int8_t* out = planes + ((int64_t)p * rows + row) * cols;
    for (int64_t col = 0; col < cols; ++col) out[col] = orc_centered_i64(src[row * ld + col], m);
  }
}

/* cpu_reference.cpp:81-107 */
void orc_pack_u64(const uint64_t* src, int64_t rows, int64_t cols, int64_t ld, uint32_t prefix, int8_t* planes) {
  const int64_t plane_rows = (int64_t)prefix * rows;
#pragma omp parallel for schedule(static)
  for (int64_t pr = 0; pr < plane_rows; ++pr) {
    const uint32_t p = (uint32_t)(pr / rows);
    const int64_t row = pr % rows;
    const uint32_t m = kLadder[p];
    int8_t* out = planes + ((int64_t)p * rows + row) * cols;
    for (int64_t col = 0; col < cols; ++col) out[col] = orc_centered_u64(src[row * ld + col], m);
  }
}

/* cpu_reference.cpp:109-130 */
void orc_pack_finite_u8(const uint8_t* src, int64_t rows, int64_t cols, int64_t ld, uint32_t modulus,
                        int8_t* plane) {
#pragma omp parallel for schedule(static)
  for (int64_t row = 0; row < rows; ++row)
    for (int64_t col = 0; col < cols; ++col)
      plane[row * cols + col] = center_canonical(src[row * ld + col] % modulus, modulus);
}

/* ---- ring GEMM ----------------------------------------------------------- */

/* cpu_reference.cpp:156-177: k-outer / col-inner int32 block accumulator */
static void ring_gemm_row(const int8_t* A, const int8_t* B, int8_t* C, int64_t n, int64_t k, int64_t lda,
                          int64_t ldb, int64_t ldc, uint32_t modulus, int64_t row, int32_t* acc) {
  int8_t* c_row = C + row * ldc;
  memset(c_row, 0, (size_t)n);
  for (int64_t offset = 0; offset < k;) {
    const int64_t block = (k - offset) < ORC_K_BLOCK ? (k - offset) : ORC_K_BLOCK;
    memset(acc, 0, sizeof(int32_t) * (size_t)n);
    for (int64_t kk = 0; kk < block; ++kk) {
      const int32_t av = A[row * lda + offset + kk];
      const int8_t* b_row = B + (offset + kk) * ldb;
      for (int64_t col = 0; col < n; ++col) acc[col] += av * (int32_t)b_row[col];
    }
    for (int64_t col = 0; col < n; ++col)
      c_row[col] = orc_reduce_to_centered((int64_t)c_row[col] + acc[col], modulus);
    offset += block;
  }
}

/* cpu_reference.cpp:188-206 (row parallel) */
void orc_ring_gemm_modulus(const int8_t* A, const int8_t* B, int8_t* C, int64_t m, int64_t n, int64_t k,
                           int64_t lda, int64_t ldb, int64_t ldc, uint32_t modulus) {
#pragma omp parallel
  {
    int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n > 0 ? n : 1));
#pragma omp for schedule(static)
    for (int64_t row = 0; row < m; ++row) ring_gemm_row(A, B, C, n, k, lda, ldb, ldc, modulus, row, acc);
    free(acc);
  }
}

/* cpu_reference.cpp:221-284 (non-tiled: every plane of the selected prefix) */
void orc_gemm_rns(const int8_t* A, const int8_t* B, int8_t* C, int64_t m, int64_t n, int64_t k,
                  uint32_t prefix) {
  for (uint32_t p = 0; p < prefix; ++p)
    orc_ring_gemm_modulus(A + (int64_t)p * m * k, B + (int64_t)p * k * n, C + (int64_t)p * m * n, m, n, k, k, n,
                          n, kLadder[p]);
}

/* residue_dot.hpp:21-38 */
int8_t orc_centered_residue_dot(const int8_t* a, const int8_t* b, int64_t k, int64_t b_stride,
                                uint32_t modulus) {
  int8_t reduced = 0;
  for (int64_t offset = 0; offset < k;) {
    const int64_t block = (k - offset) < ORC_K_BLOCK ? (k - offset) : ORC_K_BLOCK;
    int32_t acc = 0;
    for (int64_t i = offset; i < offset + block; ++i) acc += (int32_t)a[i] * (int32_t)b[i * b_stride];
    reduced = orc_reduce_to_centered((int64_t)acc + reduced, modulus);
    offset += block;
  }
  return reduced;
}

/* ---- CRT ----------------------------------------------------------------- */

/* crt.cpp:9-32 extended Euclid */
static uint32_t mod_inverse(uint32_t a, uint32_t modulus) {
  int64_t t = 0, next_t = 1, r = modulus, next_r = a % modulus;
  while (next_r != 0) {
    const int64_t q = r / next_r;
    const int64_t nt = t - q * next_t;
    t = next_t;
    next_t = nt;
    const int64_t nr = r - q * next_r;
    r = next_r;
    next_r = nr;
  }
  if (r != 1) return 0;
  if (t < 0) t += modulus;
  return (uint32_t)t;
}

/* crt.cpp:54-76 incremental Garner */
static u256 reconstruct_canonical(const int8_t* residues, int64_t stride, uint32_t prefix) {
  u256 x = u256_of(0), product = u256_of(1);
  for (uint32_t i = 0; i < prefix; ++i) {
    const uint32_t m = kLadder[i];
    const uint32_t target = orc_canonical_from_centered(residues[(int64_t)i * stride], m);
    const uint32_t x_mod = u256_mod_small(&x, m);
    const uint32_t inverse = mod_inverse(u256_mod_small(&product, m), m);
    int64_t delta = ((int64_t)target - (int64_t)x_mod) % (int64_t)m;
    if (delta < 0) delta += m;
    const uint32_t coef = (uint32_t)(((uint64_t)delta * inverse) % m);
    const u256 step = u256_mul_u64(product, coef);
    x = u256_add(x, &step);
    product = u256_mul_u64(product, m);
  }
  return x;
}

void orc_reconstruct_canonical(const int8_t* residues, uint32_t prefix, uint64_t out[4]) {
  const u256 x = reconstruct_canonical(residues, 1, prefix);
  memcpy(out, x.w, sizeof(x.w));
}

/* crt.cpp:47-50: centered representative as (negative, magnitude) */
static void centered_of(const u256* x, const u256* product, int* negative, u256* magnitude) {
  u256 threshold = u256_add(*product, &(u256){{1, 0, 0, 0}});
  /* threshold = (P + 1) / 2 */
  for (int i = 0; i < 4; ++i) {
    threshold.w[i] = (threshold.w[i] >> 1) | (i < 3 ? threshold.w[i + 1] << 63 : 0);
  }
  if (u256_cmp(x, &threshold) >= 0) {
    *negative = 1;
    *magnitude = u256_sub(*product, x);
  } else {
    *negative = 0;
    *magnitude = *x;
  }
}

/* moduli.cpp:234-293 restricted to the global bound kinds used by export */
static int bound_contract(uint32_t semantics, uint64_t bound, uint32_t prefix) {
  if (prefix == 0 || prefix > ORC_MAX_PREFIX) return ORC_INVALID_ARGUMENT;
  const u256 product = modulus_product(prefix);
  if (semantics == SEM_BOUNDED_I64) {
    if (bound > (1ull << 63)) return ORC_INVALID_ARGUMENT;
    const u256 required = u256_mul_u64(u256_of(bound), 2);
    return u256_cmp(&product, &required) > 0 ? ORC_SUCCESS : ORC_RANGE_ERROR;
  }
  const u256 required = u256_of(bound);
  return u256_cmp(&product, &required) > 0 ? ORC_SUCCESS : ORC_RANGE_ERROR;
}

static int reconstruct_signed_strided(const int8_t* residues, int64_t stride, uint32_t prefix, uint64_t bound,
                                      int64_t* out) {
  if (prefix == 0 || prefix > ORC_MAX_PREFIX) return ORC_INVALID_ARGUMENT;
  const int st = bound_contract(SEM_BOUNDED_I64, bound, prefix);
  if (st != ORC_SUCCESS) return st;
  const u256 product = modulus_product(prefix);
  const u256 x = reconstruct_canonical(residues, stride, prefix);
  int negative;
  u256 mag;
  centered_of(&x, &product, &negative, &mag);
  /* fits int64 and |v| <= bound (crt.cpp:113-119) */
  if (mag.w[1] | mag.w[2] | mag.w[3]) return ORC_RANGE_ERROR;
  if (negative ? mag.w[0] > (1ull << 63) : mag.w[0] > (uint64_t)INT64_MAX) return ORC_RANGE_ERROR;
  if (mag.w[0] > bound) return ORC_RANGE_ERROR;
  *out = negative ? (int64_t)(0 - mag.w[0]) : (int64_t)mag.w[0];
  return ORC_SUCCESS;
}

static int reconstruct_unsigned_strided(const int8_t* residues, int64_t stride, uint32_t prefix, uint64_t bound,
                                        uint64_t* out) {
  if (prefix == 0 || prefix > ORC_MAX_PREFIX) return ORC_INVALID_ARGUMENT;
  const int st = bound_contract(SEM_BOUNDED_U64, bound, prefix);
  if (st != ORC_SUCCESS) return st;
  const u256 x = reconstruct_canonical(residues, stride, prefix);
  if (x.w[1] | x.w[2] | x.w[3]) return ORC_RANGE_ERROR;
  if (x.w[0] > bound) return ORC_RANGE_ERROR;
  *out = x.w[0];
  return ORC_SUCCESS;
}

int orc_reconstruct_signed(const int8_t* residues, uint32_t prefix, uint64_t bound, int64_t* out) {
  return reconstruct_signed_strided(residues, 1, prefix, bound, out);
}

int orc_reconstruct_unsigned(const int8_t* residues, uint32_t prefix, uint64_t bound, uint64_t* out) {
  return reconstruct_unsigned_strided(residues, 1, prefix, bound, out);
}

/* crt.cpp:144-170 */
static int ew_signed_strided(const int8_t* residues, int64_t stride, uint32_t prefix, uint64_t* out,
                             uint32_t limbs) {
  if (!out || prefix == 0 || prefix > ORC_MAX_PREFIX || limbs == 0 || limbs > 32) return ORC_INVALID_ARGUMENT;
  const u256 product = modulus_product(prefix);
  const u256 x = reconstruct_canonical(residues, stride, prefix);
  int negative;
  u256 mag;
  centered_of(&x, &product, &negative, &mag);
  if (limbs < 4) {
    /* representable range [-2^(bits-1), 2^(bits-1) - 1] */
    const u256 half = u256_pow2(64u * limbs - 1u);
    if (negative ? u256_cmp(&mag, &half) > 0 : u256_cmp(&mag, &half) >= 0) return ORC_RANGE_ERROR;
  }
  u256 v = mag;
  if (negative) v = u256_sub(u256_of(0), &mag); /* two's complement over 256 bits */
  for (uint32_t l = 0; l < limbs; ++l) out[l] = l < 4 ? v.w[l] : (negative ? UINT64_MAX : 0);
  return ORC_SUCCESS;
}

/* crt.cpp:123-142 */
static int ew_unsigned_strided(const int8_t* residues, int64_t stride, uint32_t prefix, uint64_t* out,
                               uint32_t limbs) {
  if (!out || prefix == 0 || prefix > ORC_MAX_PREFIX || limbs == 0 || limbs > 32) return ORC_INVALID_ARGUMENT;
  const u256 x = reconstruct_canonical(residues, stride, prefix);
  for (uint32_t l = limbs; l < 4; ++l)
    if (x.w[l]) return ORC_RANGE_ERROR;
  for (uint32_t l = 0; l < limbs; ++l) out[l] = l < 4 ? x.w[l] : 0;
  return ORC_SUCCESS;
}

int orc_exact_wide_signed_limbs(const int8_t* residues, uint32_t prefix, uint64_t* out, uint32_t limbs) {
  return ew_signed_strided(residues, 1, prefix, out, limbs);
}

int orc_exact_wide_unsigned_limbs(const int8_t* residues, uint32_t prefix, uint64_t* out, uint32_t limbs) {
  return ew_unsigned_strided(residues, 1, prefix, out, limbs);
}

/* ---- matrix exports (api_export.cpp:365-414, 631-716): staged ---------- */

static int first_failure(const int* status, int64_t cells) {
  for (int64_t i = 0; i < cells; ++i)
    if (status[i] != ORC_SUCCESS) return status[i];
  return ORC_SUCCESS;
}

int orc_export_i64(const int8_t* C, int64_t m, int64_t n, uint32_t prefix, uint64_t bound, int64_t* dst,
                   int64_t ld) {
  const int64_t cells = m * n;
  int64_t* staged = (int64_t*)malloc(sizeof(int64_t) * (size_t)cells);
  int* status = (int*)malloc(sizeof(int) * (size_t)cells);
#pragma omp parallel for schedule(static)
  for (int64_t cell = 0; cell < cells; ++cell)
    status[cell] = reconstruct_signed_strided(C + cell, cells, prefix, bound, &staged[cell]);
  const int st = first_failure(status, cells);
  if (st == ORC_SUCCESS)
    for (int64_t r = 0; r < m; ++r) memcpy(dst + r * ld, staged + r * n, sizeof(int64_t) * (size_t)n);
  free(staged);
  free(status);
  return st;
}

int orc_export_u64(const int8_t* C, int64_t m, int64_t n, uint32_t prefix, uint64_t bound, uint64_t* dst,
                   int64_t ld) {
  const int64_t cells = m * n;
  uint64_t* staged = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)cells);
  int* status = (int*)malloc(sizeof(int) * (size_t)cells);
#pragma omp parallel for schedule(static)
  for (int64_t cell = 0; cell < cells; ++cell)
    status[cell] = reconstruct_unsigned_strided(C + cell, cells, prefix, bound, &staged[cell]);
  const int st = first_failure(status, cells);
  if (st == ORC_SUCCESS)
    for (int64_t r = 0; r < m; ++r) memcpy(dst + r * ld, staged + r * n, sizeof(uint64_t) * (size_t)n);
  free(staged);
  free(status);
  return st;
}

/* ---- per-tile bounded schedules ------------------------------------------- */

#define ORC_TILE_ZERO_OUTPUT 0x1u         /* rns8.h:74 */
#define ORC_TILE_ZERO_ROW_COL_PRODUCT 0x2u /* rns8.h:75 */
#define ORC_PLAN_FORCE_FIXED_PREFIX 0x1u
#define ORC_PLAN_ZERO_TILE_SKIPS 0x2u
#define ORC_PLAN_ZERO_ROW_COL_SKIPS 0x4u

static uint32_t u256_bit_length(const u256* v) {
  for (int i = 3; i >= 0; --i)
    if (v->w[i]) return (uint32_t)(64 * i + 64 - __builtin_clzll(v->w[i]));
  return 0;
}

static int mask_has_set(const uint8_t* mask, int64_t begin, int64_t end) {
  for (int64_t i = begin; i < end; ++i)
    if (mask[i]) return 1;
  return 0;
}

/* api_plan_schedule.inc:54-72 (make_tile_schedule_entry) */
static orc_tile_entry tile_entry(int64_t m, int64_t n, uint32_t tile_m, uint32_t tile_n, uint64_t tile_cols,
                                 uint64_t index, uint32_t required, uint32_t selected, uint32_t range_bits,
                                 uint32_t flags) {
  orc_tile_entry e;
  memset(&e, 0, sizeof(e));
  e.flags = flags;
  e.tile_row = index / tile_cols;
  e.tile_col = index % tile_cols;
  e.row_offset = (int64_t)(e.tile_row * tile_m);
  e.col_offset = (int64_t)(e.tile_col * tile_n);
  e.row_extent = (m - e.row_offset) < (int64_t)tile_m ? (m - e.row_offset) : (int64_t)tile_m;
  e.col_extent = (n - e.col_offset) < (int64_t)tile_n ? (n - e.col_offset) : (int64_t)tile_n;
  e.required_prefix = required;
  e.selected_prefix = selected;
  e.range_bit_length = range_bits;
  return e;
}

/* range of a bound: 2 * bound (signed) or bound (api_plan_schedule.inc:35-38) */
static u256 tile_range(uint32_t semantics, uint64_t bound) {
  return semantics == SEM_BOUNDED_I64 ? u256_mul_u64(u256_of(bound), 2) : u256_of(bound);
}

int orc_tile_schedule(uint32_t semantics, int64_t m, int64_t n, uint32_t tile_m, uint32_t tile_n,
                      const uint64_t* tile_bounds, uint64_t count, uint32_t budget, uint32_t flags,
                      const uint8_t* zero_a_rows, const uint8_t* zero_b_cols, orc_tile_entry* entries,
                      orc_schedule_summary* s) {
  if (semantics != SEM_BOUNDED_I64 && semantics != SEM_BOUNDED_U64) return ORC_INVALID_ARGUMENT;
  if (m <= 0 || n <= 0 || !s) return ORC_INVALID_ARGUMENT;
  if (tile_m == 0) tile_m = 128;
  if (tile_n == 0) tile_n = 128;
  memset(s, 0, sizeof(*s));
  s->tile_rows = (uint64_t)((m + tile_m - 1) / tile_m);
  s->tile_cols = (uint64_t)((n + tile_n - 1) / tile_n);
  s->tile_count = s->tile_rows * s->tile_cols;
  const int proofs = (flags & ORC_PLAN_ZERO_ROW_COL_SKIPS) != 0;
  if (proofs) {
    if (!zero_a_rows || !zero_b_cols) return ORC_INVALID_ARGUMENT;
    for (int64_t r = 0; r < m; ++r) s->zero_a_row_count += zero_a_rows[r] != 0;
    for (int64_t c = 0; c < n; ++c) s->zero_b_col_count += zero_b_cols[c] != 0;
    s->zero_row_col_product_count =
        s->zero_a_row_count * (uint64_t)n + ((uint64_t)m - s->zero_a_row_count) * s->zero_b_col_count;
  }
  if (!tile_bounds || count != s->tile_count || !entries) return ORC_INVALID_ARGUMENT;
  const int fixed = (flags & ORC_PLAN_FORCE_FIXED_PREFIX) != 0;
  const int zero_tiles = (flags & ORC_PLAN_ZERO_TILE_SKIPS) != 0;
  uint32_t min_req = UINT32_MAX, max_req = 0, min_sel = UINT32_MAX, max_sel = 0, max_bits = 0;
  uint32_t present[ORC_MAX_PREFIX + 1];
  memset(present, 0, sizeof(present));
  for (uint64_t i = 0; i < count; ++i) {
    const uint64_t bound = tile_bounds[i];
    if (semantics == SEM_BOUNDED_I64 && bound > (1ull << 63)) return ORC_INVALID_ARGUMENT;
    const u256 range = tile_range(semantics, bound);
    const uint32_t bits = u256_bit_length(&range);
    const uint32_t req = required_prefix(&range);
    if (req == 0 || req > budget) return ORC_RANGE_ERROR;
    const uint32_t sel = fixed ? budget : req;
    min_req = req < min_req ? req : min_req;
    max_req = req > max_req ? req : max_req;
    min_sel = sel < min_sel ? sel : min_sel;
    max_sel = sel > max_sel ? sel : max_sel;
    max_bits = bits > max_bits ? bits : max_bits;
    present[sel] = 1;
    uint32_t ef = zero_tiles && bound == 0 ? ORC_TILE_ZERO_OUTPUT : 0u;
    orc_tile_entry e = tile_entry(m, n, tile_m, tile_n, s->tile_cols, i, req, sel, bits, 0);
    if (proofs && (mask_has_set(zero_a_rows, e.row_offset, e.row_offset + e.row_extent) ||
                   mask_has_set(zero_b_cols, e.col_offset, e.col_offset + e.col_extent)))
      ef |= ORC_TILE_ZERO_ROW_COL_PRODUCT;
    e.flags = ef;
    s->flags |= ef;
    entries[i] = e;
  }
  /* group index = rank of the selected prefix among the distinct ones */
  uint32_t rank[ORC_MAX_PREFIX + 1];
  uint32_t groups = 0;
  for (uint32_t p = 0; p <= ORC_MAX_PREFIX; ++p) {
    rank[p] = groups;
    groups += present[p];
  }
  for (uint64_t i = 0; i < count; ++i) entries[i].group_index = rank[entries[i].selected_prefix];
  s->min_required = count ? min_req : 0;
  s->max_required = max_req;
  s->min_selected = count ? min_sel : 0;
  s->max_selected = max_sel;
  s->group_count = groups;
  s->range_bits = max_bits;
  s->adaptive_prefix = groups > 1;
  s->adaptive_skip = max_sel < budget;
  s->collapsed = groups == 1 && min_req == budget && max_req == budget && min_sel == budget && max_sel == budget &&
                 s->flags == 0;
  if (s->collapsed) {
    /* api_plan_public_api.inc:141-157: entries rebuilt from the copied bounds */
    for (uint64_t i = 0; i < count; ++i) {
      const u256 range = tile_range(semantics, tile_bounds[i]);
      entries[i] = tile_entry(m, n, tile_m, tile_n, s->tile_cols, i, required_prefix(&range), s->min_selected,
                              u256_bit_length(&range), 0);
    }
  }
  return ORC_SUCCESS;
}

void orc_gemm_rns_tiled(const int8_t* A, const int8_t* B, int8_t* C, int64_t m, int64_t n, int64_t k,
                        const orc_tile_entry* entries, uint64_t count) {
  for (uint64_t t = 0; t < count; ++t) {
    const orc_tile_entry* e = &entries[t];
    for (uint32_t p = 0; p < e->selected_prefix; ++p) {
      int8_t* c_tile = C + (int64_t)p * m * n + e->row_offset * n + e->col_offset;
      if (e->flags & ORC_TILE_ZERO_OUTPUT) {
        for (int64_t r = 0; r < e->row_extent; ++r) memset(c_tile + r * n, 0, (size_t)e->col_extent);
        continue;
      }
      orc_ring_gemm_modulus(A + (int64_t)p * m * k + e->row_offset * k, B + (int64_t)p * k * n + e->col_offset,
                            c_tile, e->row_extent, e->col_extent, k, k, n, n, kLadder[p]);
    }
  }
}

static const orc_tile_entry* entry_for_cell(const orc_tile_entry* entries, uint64_t count, uint32_t tile_m,
                                            uint32_t tile_n, int64_t n, int64_t row, int64_t col) {
  const uint64_t cols = (uint64_t)((n + tile_n - 1) / tile_n);
  const uint64_t index = (uint64_t)(row / tile_m) * cols + (uint64_t)(col / tile_n);
  return index < count ? &entries[index] : NULL;
}

int orc_export_i64_tiled(const int8_t* C, int64_t m, int64_t n, uint32_t storage, uint32_t tile_m, uint32_t tile_n,
                         const orc_tile_entry* entries, const uint64_t* tile_bounds, uint64_t count, int64_t* dst,
                         int64_t ld) {
  const int64_t cells = m * n;
  int64_t* staged = (int64_t*)calloc((size_t)cells, sizeof(int64_t));
  int* status = (int*)calloc((size_t)cells, sizeof(int));
  (void)storage;
#pragma omp parallel for schedule(static)
  for (int64_t cell = 0; cell < cells; ++cell) {
    const int64_t row = cell / n, col = cell % n;
    const orc_tile_entry* e = entry_for_cell(entries, count, tile_m, tile_n, n, row, col);
    if (!e) { status[cell] = ORC_INVALID_ARGUMENT; continue; }
    if (e->flags & ORC_TILE_ZERO_OUTPUT) { staged[cell] = 0; continue; }
    const uint64_t idx = (uint64_t)(e - entries);
    status[cell] = reconstruct_signed_strided(C + cell, cells, e->selected_prefix, tile_bounds[idx], &staged[cell]);
  }
  const int st = first_failure(status, cells);
  if (st == ORC_SUCCESS)
    for (int64_t r = 0; r < m; ++r) memcpy(dst + r * ld, staged + r * n, sizeof(int64_t) * (size_t)n);
  free(staged);
  free(status);
  return st;
}

int orc_export_u64_tiled(const int8_t* C, int64_t m, int64_t n, uint32_t storage, uint32_t tile_m, uint32_t tile_n,
                         const orc_tile_entry* entries, const uint64_t* tile_bounds, uint64_t count, uint64_t* dst,
                         int64_t ld) {
  const int64_t cells = m * n;
  uint64_t* staged = (uint64_t*)calloc((size_t)cells, sizeof(uint64_t));
  int* status = (int*)calloc((size_t)cells, sizeof(int));
  (void)storage;
#pragma omp parallel for schedule(static)
  for (int64_t cell = 0; cell < cells; ++cell) {
    const int64_t row = cell / n, col = cell % n;
    const orc_tile_entry* e = entry_for_cell(entries, count, tile_m, tile_n, n, row, col);
    if (!e) { status[cell] = ORC_INVALID_ARGUMENT; continue; }
    if (e->flags & ORC_TILE_ZERO_OUTPUT) { staged[cell] = 0; continue; }
    const uint64_t idx = (uint64_t)(e - entries);
    status[cell] =
        reconstruct_unsigned_strided(C + cell, cells, e->selected_prefix, tile_bounds[idx], &staged[cell]);
  }
  const int st = first_failure(status, cells);
  if (st == ORC_SUCCESS)
    for (int64_t r = 0; r < m; ++r) memcpy(dst + r * ld, staged + r * n, sizeof(uint64_t) * (size_t)n);
  free(staged);
  free(status);
  return st;
}

static int export_limbs(const int8_t* C, int64_t m, int64_t n, uint32_t prefix, uint64_t* dst, int64_t ld,
                        uint32_t limbs, int is_signed) {
  const int64_t cells = m * n;
  uint64_t* staged = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)cells * limbs);
  int* status = (int*)malloc(sizeof(int) * (size_t)cells);
#pragma omp parallel for schedule(static)
  for (int64_t cell = 0; cell < cells; ++cell)
    status[cell] = is_signed ? ew_signed_strided(C + cell, cells, prefix, staged + cell * limbs, limbs)
                             : ew_unsigned_strided(C + cell, cells, prefix, staged + cell * limbs, limbs);
  const int st = first_failure(status, cells);
  if (st == ORC_SUCCESS)
    for (int64_t r = 0; r < m; ++r)
      memcpy(dst + r * ld * limbs, staged + r * n * limbs, sizeof(uint64_t) * (size_t)(n * limbs));
  free(staged);
  free(status);
  return st;
}

int orc_export_exact_wide_signed(const int8_t* C, int64_t m, int64_t n, uint32_t prefix, uint64_t* dst, int64_t ld,
                                 uint32_t limbs) {
  return export_limbs(C, m, n, prefix, dst, ld, limbs, 1);
}

int orc_export_exact_wide_unsigned(const int8_t* C, int64_t m, int64_t n, uint32_t prefix, uint64_t* dst,
                                   int64_t ld, uint32_t limbs) {
  return export_limbs(C, m, n, prefix, dst, ld, limbs, 0);
}

/* cpu_reference.cpp:132-153 */
void orc_export_finite_u8(const int8_t* C, int64_t m, int64_t n, uint32_t modulus, uint8_t* dst, int64_t ld) {
  for (int64_t r = 0; r < m; ++r)
    for (int64_t c = 0; c < n; ++c) dst[r * ld + c] = (uint8_t)orc_canonical_from_centered(C[r * n + c], modulus);
}

/* ---- end-to-end sample paths ------------------------------------------- */

int orc_gemm_i64_rows(const int64_t* A, int64_t lda, const int64_t* B, int64_t ldb, int64_t k, int64_t n,
                      int64_t row0, int64_t rows, uint32_t prefix, uint64_t bound, int64_t* C, int64_t ldc) {
  int8_t* ap = (int8_t*)malloc((size_t)prefix * rows * k);
  int8_t* bp = (int8_t*)malloc((size_t)prefix * k * n);
  int8_t* cp = (int8_t*)malloc((size_t)prefix * rows * n);
  orc_pack_i64(A + row0 * lda, rows, k, lda, prefix, ap);
  orc_pack_i64(B, k, n, ldb, prefix, bp);
  orc_gemm_rns(ap, bp, cp, rows, n, k, prefix);
  const int st = orc_export_i64(cp, rows, n, prefix, bound, C, ldc);
  free(ap);
  free(bp);
  free(cp);
  return st;
}

int orc_gemm_u64_rows(const uint64_t* A, int64_t lda, const uint64_t* B, int64_t ldb, int64_t k, int64_t n,
                      int64_t row0, int64_t rows, uint32_t prefix, uint64_t bound, uint64_t* C, int64_t ldc) {
  int8_t* ap = (int8_t*)malloc((size_t)prefix * rows * k);
  int8_t* bp = (int8_t*)malloc((size_t)prefix * k * n);
  int8_t* cp = (int8_t*)malloc((size_t)prefix * rows * n);
  orc_pack_u64(A + row0 * lda, rows, k, lda, prefix, ap);
  orc_pack_u64(B, k, n, ldb, prefix, bp);
  orc_gemm_rns(ap, bp, cp, rows, n, k, prefix);
  const int st = orc_export_u64(cp, rows, n, prefix, bound, C, ldc);
  free(ap);
  free(bp);
  free(cp);
  return st;
}

void orc_gemm_finite_u8_rows(const uint8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, int64_t k, int64_t n,
                             int64_t row0, int64_t rows, uint32_t modulus, uint8_t* C, int64_t ldc) {
  int8_t* ap = (int8_t*)malloc((size_t)rows * k);
  int8_t* bp = (int8_t*)malloc((size_t)k * n);
  int8_t* cp = (int8_t*)malloc((size_t)rows * n);
  orc_pack_finite_u8(A + row0 * lda, rows, k, lda, modulus, ap);
  orc_pack_finite_u8(B, k, n, ldb, modulus, bp);
  orc_ring_gemm_modulus(ap, bp, cp, rows, n, k, k, n, n, modulus);
  orc_export_finite_u8(cp, rows, n, modulus, C, ldc);
  free(ap);
  free(bp);
  free(cp);
}

int orc_gemm_exact_wide_signed_rows(const int64_t* A, int64_t lda, const int64_t* B, int64_t ldb, int64_t k,
                                    int64_t n, int64_t row0, int64_t rows, uint32_t prefix, uint64_t* C,
                                    int64_t ldc, uint32_t limbs) {
  int8_t* ap = (int8_t*)malloc((size_t)prefix * rows * k);
  int8_t* bp = (int8_t*)malloc((size_t)prefix * k * n);
  int8_t* cp = (int8_t*)malloc((size_t)prefix * rows * n);
  orc_pack_i64(A + row0 * lda, rows, k, lda, prefix, ap);
  orc_pack_i64(B, k, n, ldb, prefix, bp);
  orc_gemm_rns(ap, bp, cp, rows, n, k, prefix);
  const int st = orc_export_exact_wide_signed(cp, rows, n, prefix, C, ldc, limbs);
  free(ap);
  free(bp);
  free(cp);
  return st;
}

/* ---- brute-force exact GEMM --------------------------------------------- */

static void store_limbs(const u256* v, int negative_fill, uint64_t* out, uint32_t limbs) {
  for (uint32_t l = 0; l < limbs; ++l) out[l] = l < 4 ? v->w[l] : (negative_fill ? UINT64_MAX : 0);
}

void orc_exact_gemm_i64(const int64_t* A, int64_t lda, const int64_t* B, int64_t ldb, int64_t m, int64_t n,
                        int64_t k, uint64_t* C, int64_t ldc, uint32_t limbs) {
#pragma omp parallel for schedule(static)
  for (int64_t cell = 0; cell < m * n; ++cell) {
    const int64_t r = cell / n, c = cell % n;
    u256 acc = u256_of(0);
    for (int64_t kk = 0; kk < k; ++kk) {
      const __int128 prod = (__int128)A[r * lda + kk] * (__int128)B[kk * ldb + c];
      const uint64_t fill = prod < 0 ? UINT64_MAX : 0;
      const u256 term = {{(uint64_t)prod, (uint64_t)((unsigned __int128)prod >> 64), fill, fill}};
      acc = u256_add(acc, &term);
    }
    store_limbs(&acc, (acc.w[3] >> 63) != 0, C + (r * ldc + c) * limbs, limbs);
  }
}

void orc_exact_gemm_u64(const uint64_t* A, int64_t lda, const uint64_t* B, int64_t ldb, int64_t m, int64_t n,
                        int64_t k, uint64_t* C, int64_t ldc, uint32_t limbs) {
#pragma omp parallel for schedule(static)
  for (int64_t cell = 0; cell < m * n; ++cell) {
    const int64_t r = cell / n, c = cell % n;
    u256 acc = u256_of(0);
    for (int64_t kk = 0; kk < k; ++kk) {
      const unsigned __int128 prod = (unsigned __int128)A[r * lda + kk] * B[kk * ldb + c];
      const u256 term = {{(uint64_t)prod, (uint64_t)(prod >> 64), 0, 0}};
      acc = u256_add(acc, &term);
    }
    store_limbs(&acc, 0, C + (r * ldc + c) * limbs, limbs);
  }
}

/* ---- seeded inputs -------------------------------------------------------- */

#define SPLITMIX_GAMMA 0x9e3779b97f4a7c15ull

static uint64_t splitmix_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

uint64_t orc_splitmix64_next(uint64_t* state) {
  *state += SPLITMIX_GAMMA;
  return splitmix_mix(*state);
}

void orc_fill(uint64_t seed, uint32_t mode, uint32_t bits_or_limit, void* out, int64_t count) {
  if (mode == 3) {
    uint8_t* o = (uint8_t*)out;
    uint64_t state = seed;
    for (int64_t i = 0; i < count;) {
      const uint64_t x = orc_splitmix64_next(&state);
      const uint32_t byte = (uint32_t)(x & 0xffu);
      if (byte < bits_or_limit) o[i++] = (uint8_t)byte;
    }
    return;
  }
  uint64_t* o = (uint64_t*)out;
  const uint32_t b = bits_or_limit;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < count; ++i) {
    const uint64_t x = splitmix_mix(seed + (uint64_t)(i + 1) * SPLITMIX_GAMMA);
    if (mode == 0) {
      o[i] = (uint64_t)((int64_t)(x >> (63u - b)) - (int64_t)(1ull << b));
    } else if (mode == 1) {
      o[i] = b >= 64 ? x : (x >> (64u - b));
    } else {
      o[i] = x;
    }
  }
}

/* rns8_bench_support.cpp:96-99 and rns8_bench_event_phase_helpers.inc:544-552 */
uint64_t orc_checksum_u64(const uint64_t* values, int64_t rows, int64_t cols, int64_t ld, uint32_t limbs) {
  uint64_t h = 1469598103934665603ull;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c)
      for (uint32_t l = 0; l < limbs; ++l) {
        h ^= values[(r * ld + c) * limbs + l];
        h *= 1099511628211ull;
      }
  return h;
}

uint64_t orc_checksum_u8(const uint8_t* values, int64_t rows, int64_t cols, int64_t ld) {
  uint64_t h = 1469598103934665603ull;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      h ^= values[r * ld + c];
      h *= 1099511628211ull;
    }
  return h;
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void orc_set_num_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
}
