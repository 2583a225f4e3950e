// Constant tables shared by the host runtime and the gfx950 kernels.
//
// Everything the kernels need per modulus is precomputed here on the host and
// passed by value as kernel arguments (uniform values land in SGPRs). The
// arithmetic identities behind each table are stated next to it; tests in
// tests/test_tables.py check them exhaustively on the CPU.
#pragma once

#include <cstdint>

namespace rns8x {

// Modulus ladder (reference src/core/internal.hpp:328-330): 28 pairwise-coprime
// moduli <= 256; prefixes of at most 20 are used.
constexpr uint32_t kLadderSize = 28;
constexpr uint32_t kMaxPrefix = 20;
constexpr uint16_t kLadder[kLadderSize] = {256, 255, 253, 251, 247, 239, 233, 229, 227, 223,
                                           217, 211, 199, 197, 193, 191, 181, 179, 173, 167,
                                           163, 157, 151, 149, 139, 137, 131, 127};

// int8 x int8 products are at most 2^14 in magnitude, so 65536 of them plus a
// carried centered residue fit in int32 (reference residue_dot.hpp:18-19).
constexpr int64_t kSafeKBlock = 65536;

// ---- exact small-modulus reduction ---------------------------------------
//
// For 2 <= m <= 256 let R = ceil(2^32 / m) and e = R*m - 2^32 (0 <= e < m).
// For 0 <= s < 2^21, floor(s*R / 2^32) == floor(s / m) because s*e < 2^29 <
// 2^32 keeps the error term below 1/m. So q = umulhi(s, R), r = s - q*m.
//
// Centering: with H = floor(m/2), centered(x) = ((x + H) mod m) - H equals the
// reference rule "r >= (m+1)/2 ? r - m : r" (cpu_reference.cpp:26-32) for
// every m >= 2. H is folded into the additive offsets below.
struct ModulusConsts {
  uint32_t m;
  uint32_t half;    // H = floor(m/2)
  uint32_t recip;   // R = ceil(2^32 / m)
  uint32_t pow_lo;  // bytes [2^0, 2^8, 2^16, 2^24] mod m, packed little-endian
  uint32_t pow_hi;  // bytes [2^32, 2^40, 2^48, 2^56] mod m
  uint32_t off_i64; // H + (-2^63 mod m): int64 x read as u = x ^ 2^63
  uint32_t off_u64; // H
  uint32_t off_i32; // H + (-2^31 mod m): int32 acc read as u = acc + 2^31
  // Full-rate quotient for the int32 reduction: s = dot(bytes(u), pow_lo) +
  // off_i32 never exceeds s_max = 255 * (sum of pow_lo bytes) + off_i32, and
  // floor(s / m) = mulhi_u24(s << q_shift, q_recip) (make_quot24).
  uint32_t q_shift;
  uint32_t q_recip;
  // Same for the pack reduction of a 64-bit value: s = dot(lo bytes, pow_lo)
  // + dot(hi bytes, pow_hi) + off (off_i64 or off_u64) is at most
  // 255 * (sum of pow_lo and pow_hi bytes) + max(off_i64, off_u64) < 2^19.
  uint32_t pq_shift;
  uint32_t pq_recip;
};

// Shift and reciprocal for floor(s / m) = hi32((s << a) * R) over 0 <= s <=
// s_max < 2^24, with both factors below 2^24 so v_mul_hi_u32_u24 (full rate)
// computes it. a is the largest shift with s_max * 2^a < 2^24 and
// R = ceil(2^k / m), k = 32 - a. Writing e = R*m - 2^k (0 <= e < m) and
// s = q*m + r: s*R / 2^k = q + (r + s*e / 2^k) / m, and s*e < s_max * m <=
// 2^k because s_max * 2^a * m < 2^24 * 2^8. So the floor is q. R stays below
// 2^24: maximality of a gives 2^k <= 2^9 * s_max, so R <= 2^9 * s_max / m + 1.
struct Quot24 {
  uint32_t shift;
  uint32_t recip;
};
constexpr Quot24 make_quot24(uint32_t m, uint32_t s_max) {
  uint32_t a = 0;
  while ((uint64_t{s_max} << (a + 1)) < (uint64_t{1} << 24)) ++a;
  const uint64_t k = uint64_t{1} << (32 - a);
  return Quot24{a, static_cast<uint32_t>((k + m - 1) / m)};
}

// Division by a runtime divisor d >= 1 of any n < 2^31 with one 32-bit
// high multiply (uniform values: the scalar unit's s_mul_hi_u32), no special
// cases. With s = ceil(log2 d), mul = ceil(2^(31+s) / d) <= 2^31 for d = 2^s
// and < 2^32 otherwise (d > 2^(s-1)); e = mul*d - 2^(31+s) < d gives
// n*mul / 2^(31+s) = n/d + n*e / (d 2^(31+s)) with an error term below
// n / 2^(31+s) < 2^-s <= 1/d, so floor(n / d) = floor(n*mul / 2^(31+s))
// = hi32(2n * mul) >> s (2n < 2^32; nested floors by powers of two compose).
struct DivU31 {
  uint32_t d;
  uint32_t mul;
  uint32_t shift;
};
constexpr DivU31 make_div_u31(uint32_t d) {
  if (d == 0) d = 1;
  uint32_t s = 0;
  while ((uint64_t{1} << s) < d) ++s;
  const uint64_t mul = ((uint64_t{1} << (31 + s)) + d - 1) / d;
  return DivU31{d, static_cast<uint32_t>(mul), s};
}
constexpr uint32_t div_u31_host(uint32_t n, DivU31 v) {
  return static_cast<uint32_t>((static_cast<uint64_t>(n << 1) * v.mul) >> 32) >> v.shift;
}

inline ModulusConsts make_modulus_consts(uint32_t m) {
  ModulusConsts c{};
  c.m = m;
  c.half = m / 2u;
  c.recip = static_cast<uint32_t>(((uint64_t{1} << 32) + m - 1u) / m);
  uint32_t lo = 0, hi = 0;
  for (uint32_t b = 0; b < 4; ++b) {
    const uint64_t plo = (uint64_t{1} << (8u * b)) % m;
    // 2^(32+8b) mod m computed without overflow
    uint64_t phi = (uint64_t{1} << 32) % m;
    phi = (phi * ((uint64_t{1} << (8u * b)) % m)) % m;
    lo |= static_cast<uint32_t>(plo) << (8u * b);
    hi |= static_cast<uint32_t>(phi) << (8u * b);
  }
  c.pow_lo = lo;
  c.pow_hi = hi;
  const uint64_t two63_mod = (uint64_t{1} << 63) % m;
  const uint64_t two31_mod = (uint64_t{1} << 31) % m;
  c.off_i64 = c.half + static_cast<uint32_t>((m - two63_mod) % m);
  c.off_u64 = c.half;
  c.off_i32 = c.half + static_cast<uint32_t>((m - two31_mod) % m);
  uint32_t byte_sum = 0;
  for (uint32_t b = 0; b < 4; ++b) byte_sum += (lo >> (8u * b)) & 0xFFu;
  const Quot24 q = make_quot24(m, 255u * byte_sum + c.off_i32);
  c.q_shift = q.shift;
  c.q_recip = q.recip;
  uint32_t hi_sum = 0;
  for (uint32_t b = 0; b < 4; ++b) hi_sum += (hi >> (8u * b)) & 0xFFu;
  const uint32_t off_max = c.off_i64 > c.off_u64 ? c.off_i64 : c.off_u64;
  const Quot24 pq = make_quot24(m, 255u * (byte_sum + hi_sum) + off_max);
  c.pq_shift = pq.shift;
  c.pq_recip = pq.recip;
  return c;
}

// Up to kMaxPrefix planes of modulus constants, passed by value to kernels.
struct PlaneConsts {
  ModulusConsts mod[kMaxPrefix];
};

inline PlaneConsts make_ladder_plane_consts(uint32_t prefix) {
  PlaneConsts pc{};
  for (uint32_t p = 0; p < prefix && p < kMaxPrefix; ++p) pc.mod[p] = make_modulus_consts(kLadder[p]);
  return pc;
}

inline PlaneConsts make_single_plane_consts(uint32_t modulus) {
  PlaneConsts pc{};
  pc.mod[0] = make_modulus_consts(modulus);
  return pc;
}

// ---- Garner reconstruction ---------------------------------------------------
//
// Mixed-radix digits v_i in [0, m_i) with x = sum_i v_i * P_i, P_i = prod_{t<i} m_t:
//   v_i = (r_i * I_i + sum_{j<i} v_j * W[j][i]) mod m_i
// where r_i is the centered residue, I_i = P_i^{-1} mod m_i and
// W[j][i] = (-P_j * I_i) mod m_i. This is Garner's recurrence
// v_i = (r_i - x_i) * P_i^{-1} mod m_i with x_i mod m_i expanded over the
// earlier digits, so each digit costs one reduction. Digits are kept packed
// four per dword, so the inner sum is a byte dot product (v_dot4_u32_u8) against
// wpack[i][q] = bytes W[4q..4q+3][i]. The sum stays below 2^21 (r_i*I_i + bias
// <= 2^16, 19 * 255 * 255 < 2^21), inside the exact range of the reduction
// above.
//
// The integer x is then rebuilt by Horner's rule x = (..(v_{P-1} m_{P-2} +
// v_{P-2}) m_{P-3} + ..) m_0 + v_0 in 24-bit limbs (v_mad_u32_u24 keeps every
// step exact in 32 bits).
constexpr uint32_t kGarnerDigitWords = (kMaxPrefix + 3) / 4;  // 5
constexpr uint32_t kWideLimbs = 7;                            // 7 * 24 = 168 >= 154.85 bits

struct GarnerConsts {
  uint32_t prefix;
  uint32_t m[kMaxPrefix];
  uint32_t recip[kMaxPrefix];
  uint32_t inv[kMaxPrefix];   // I_i
  uint32_t bias[kMaxPrefix];  // multiple of m_i >= 128 * I_i (keeps r_i*I_i + bias >= 0)
  uint32_t wpack[kMaxPrefix][kGarnerDigitWords];
  uint32_t half_ceil[kWideLimbs];  // ceil(P/2) = (P+1)/2 in 24-bit limbs
  uint32_t product[kWideLimbs];    // P in 24-bit limbs
};

// Simple multiprecision helper on 24-bit limbs used only to build the tables.
struct Limbs24 {
  uint32_t w[kWideLimbs] = {};
  constexpr void mul_add(uint32_t mul, uint32_t add) {
    uint64_t carry = add;
    for (uint32_t i = 0; i < kWideLimbs; ++i) {
      const uint64_t t = static_cast<uint64_t>(w[i]) * mul + carry;
      w[i] = static_cast<uint32_t>(t & 0xFFFFFFu);
      carry = t >> 24;
    }
  }
  constexpr uint32_t mod_small(uint32_t m) const {
    uint64_t r = 0;
    for (int i = static_cast<int>(kWideLimbs) - 1; i >= 0; --i) r = ((r << 24) | w[i]) % m;
    return static_cast<uint32_t>(r);
  }
};

constexpr uint32_t inverse_mod(uint32_t a, uint32_t m) {
  // extended Euclid; a and m coprime
  int64_t t = 0, nt = 1, r = m, nr = a % m;
  while (nr != 0) {
    const int64_t q = r / nr;
    const int64_t tt = t - q * nt;
    t = nt;
    nt = tt;
    const int64_t rr = r - q * nr;
    r = nr;
    nr = rr;
  }
  if (r != 1) return 0;
  if (t < 0) t += m;
  return static_cast<uint32_t>(t);
}

constexpr GarnerConsts make_garner_consts(uint32_t prefix) {
  GarnerConsts g{};
  g.prefix = prefix;
  Limbs24 pj[kMaxPrefix + 1];
  pj[0].w[0] = 1;
  for (uint32_t j = 0; j < prefix; ++j) {
    pj[j + 1] = pj[j];
    pj[j + 1].mul_add(kLadder[j], 0);
  }
  for (uint32_t i = 0; i < prefix; ++i) {
    const uint32_t m = kLadder[i];
    g.m[i] = m;
    g.recip[i] = static_cast<uint32_t>(((uint64_t{1} << 32) + m - 1u) / m);
    const uint32_t inv = i == 0 ? 1u : inverse_mod(pj[i].mod_small(m), m);
    g.inv[i] = inv;
    g.bias[i] = m * ((128u * inv + m - 1u) / m);
    for (uint32_t j = 0; j < i; ++j) {
      const uint32_t pm = pj[j].mod_small(m);
      const uint32_t w = (m - static_cast<uint32_t>((static_cast<uint64_t>(pm) * inv) % m)) % m;
      g.wpack[i][j / 4] |= w << (8u * (j % 4));
    }
  }
  // P and ceil(P/2) = (P + 1) >> 1
  Limbs24 p = pj[prefix];
  for (uint32_t i = 0; i < kWideLimbs; ++i) g.product[i] = p.w[i];
  Limbs24 h = p;
  h.mul_add(1, 1);
  for (uint32_t i = 0; i < kWideLimbs; ++i) {
    const uint32_t next = i + 1 < kWideLimbs ? h.w[i + 1] : 0u;
    g.half_ceil[i] = (h.w[i] >> 1) | ((next & 1u) << 23);
  }
  return g;
}

// ---- per-prefix Garner tables for the export kernels ----------------------------
//
// Digit i of the mixed-radix form is v_i = s mod m_i with
//   s = (r_i + 128) * I_i + xbias_i + sum_{j<i} v_j * W[j][i]
// where r_i + 128 is the residue byte with its top bit flipped (an unsigned
// byte, so the whole sum is one chain of v_dot4_u32_u8 with I_i placed at the
// cell's byte) and xbias_i = (-128 I_i) mod m_i restores r_i * I_i. With
// 0 <= s <= s_max_i the quotient comes from the full-rate 24-bit reciprocal
// of make_quot24 and v_i is the low byte of s + q*(256 - m_i) (congruent to
// s - q*m_i modulo 256, and s - q*m_i < 256).
template <uint32_t P>
struct GarnerTable {
  static constexpr uint32_t kWords = (P + 3) / 4;
  uint32_t m[P];
  uint32_t inv[P];    // I_i
  uint32_t xbias[P];
  uint32_t wpack[P][kWords == 0 ? 1 : kWords];
  uint32_t qshift[P];
  uint32_t qrecip[P];
  uint32_t active[P];  // 24-bit limbs of prod_{k >= i} m_k (Horner step i)
  uint32_t product[kWideLimbs];
  uint32_t half_ceil[kWideLimbs];
  uint32_t limbs;      // limbs of P itself
};

template <uint32_t P>
constexpr GarnerTable<P> make_garner_table() {
  const GarnerConsts g = make_garner_consts(P);
  GarnerTable<P> t{};
  for (uint32_t i = 0; i < P; ++i) {
    t.m[i] = g.m[i];
    t.inv[i] = g.inv[i];
    t.xbias[i] = (g.m[i] - (128u * g.inv[i]) % g.m[i]) % g.m[i];
    uint32_t s_max = 255u * g.inv[i] + t.xbias[i];
    for (uint32_t q = 0; q < GarnerTable<P>::kWords; ++q) {
      t.wpack[i][q] = g.wpack[i][q];
      for (uint32_t b = 0; b < 4; ++b) s_max += 255u * ((g.wpack[i][q] >> (8 * b)) & 0xFFu);
    }
    const Quot24 qq = make_quot24(g.m[i], s_max);
    t.qshift[i] = qq.shift;
    t.qrecip[i] = qq.recip;
    Limbs24 tail;
    tail.w[0] = 1;
    for (uint32_t k = i; k < P; ++k) tail.mul_add(g.m[k], 0);
    uint32_t n = 1;
    for (uint32_t l = 0; l < kWideLimbs; ++l)
      if (tail.w[l] != 0) n = l + 1;
    t.active[i] = n;
  }
  t.limbs = 1;
  for (uint32_t l = 0; l < kWideLimbs; ++l) {
    t.product[l] = g.product[l];
    t.half_ceil[l] = g.half_ceil[l];
    if (g.product[l] != 0) t.limbs = l + 1;
  }
  return t;
}

// Product of the first j ladder moduli, for products below 2^64.
constexpr uint64_t ladder_product64(uint32_t j) {
  uint64_t p = 1;
  for (uint32_t i = 0; i < j; ++i) p *= kLadder[i];
  return p;
}

// Digit splits of the 64-bit exports. An admissible int64 result has
// |v| <= 2^63 < M_J (M_j = product of the first j moduli, J = kSplitSigned),
// so its mixed-radix digits from J up are all 0 (v >= 0) or all m_i - 1
// (v < 0, x = P - |v|, no borrow past digit J - 1); an admissible uint64
// result is below 2^64 <= M_J' (J' = kSplitUnsigned), so its digits from J'
// up are all 0. Only the low J (J') digits need Horner's rule.
constexpr uint32_t split_signed() {
  uint32_t j = 0;
  while (ladder_product64(j) <= (uint64_t{1} << 63)) ++j;
  return j;
}
constexpr uint32_t kSplitSigned = split_signed();
constexpr uint32_t kSplitUnsigned = kSplitSigned + 1;  // M_{J+1} >= 2 M_J > 2^64
static_assert(kSplitSigned == 8 && ladder_product64(8) == 13057518384392951040ull, "ladder split");

// 64-bit value as 24-bit limbs.
inline void u64_to_limbs24(uint64_t v, uint32_t out[kWideLimbs]) {
  for (uint32_t i = 0; i < kWideLimbs; ++i) {
    out[i] = i < 3 ? static_cast<uint32_t>((v >> (24u * i)) & 0xFFFFFFu) : 0u;
  }
}

// ---- byte-matrix planes in HBM -------------------------------------------------
//
// Resident layout "rns8_mi355x_planes_v1": plane p of a rows x cols matrix is
// row-major int8 with a row pitch padded to 16 bytes (zero filled) and a plane
// pitch padded to 256 bytes. Padding keeps every 16-byte vector access of the
// GEMM and pack kernels aligned; the zero columns contribute nothing to any
// product, so GEMM tiles may read them freely.
constexpr int64_t kRowAlign = 16;
constexpr int64_t kPlaneAlign = 256;

// Row pitch of a plane: cols rounded up to kRowAlign (saturating at the
// largest such multiple for column counts near INT64_MAX, which no storage
// can hold; plane_pitch refuses them).
inline int64_t padded_ld(int64_t cols) {
  if (cols > INT64_MAX - (kRowAlign - 1)) return INT64_MAX / kRowAlign * kRowAlign;
  return (cols + (kRowAlign - 1)) / kRowAlign * kRowAlign;
}
// Bytes of one plane, or -1 when rows x padded_ld(cols), rounded up to
// kPlaneAlign, is not representable (the caller reports RNS8_RANGE_ERROR).
inline int64_t plane_pitch(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0 || cols > INT64_MAX - (kRowAlign - 1)) return -1;
  const int64_t ld = padded_ld(cols);
  if (rows > (INT64_MAX - (kPlaneAlign - 1)) / ld) return -1;
  const int64_t bytes = rows * ld;
  return (bytes + (kPlaneAlign - 1)) / kPlaneAlign * kPlaneAlign;
}

}  // namespace rns8x
