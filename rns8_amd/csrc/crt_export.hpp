// CRT-basis reconstruction for the MFMA export kernels: tables and the
// per-cell integer tail, shared by the gfx950 kernels (export.hip) and the
// host checks of tests/tables_check.cpp.
//
// With K_i the CRT basis element of modulus m_i over the first P ladder
// moduli (K_i = 1 mod m_i, 0 mod every other m_j, 0 <= K_i < M, M = prod m_i),
// every integer x with residues r_i satisfies
//   x = X' (mod M),   X' = sum_i r_i K_i,
// for any representatives r_i, in particular the centered int8 residues the
// planes hold. X' is a matrix product: write K_i in signed base-256 digits
// d_{i,b} in [-128, 127] (b < kDigits); then
//   X' = sum_b 256^b S_b,   S_b = sum_i r_i d_{i,b},
// and S_b (|S_b| <= 20 * 128 * 128 < 2^19) is one int8 MFMA over the planes
// (K dimension) and digit columns (N dimension) for 32 cells at a time.
//
// The centered value is v = X' - q M with q = round(X' / M). Two more MFMA
// columns hold the signed base-256 digits of F_i = round(2^kCrtFracBits K_i / M),
// so E = sum_i r_i F_i = 2^kCrtFracBits X'/M + err with |err| <= 20 * 128 / 2
// = 1280 = 0.078 * 2^kCrtFracBits, and q' = round(E / 2^kCrtFracBits) equals
// round(X'/M) unless the fraction of X'/M lies within 0.078 of one half, i.e.
// unless |v| > 0.42 M. Whatever q', |q' - round(X'/M)| <= 1, so
// v' = X' - q' M is v, v + M or v - M, and |v'| < M/2 implies v' = v (the
// exact centered range is [-M/2, M/2) because M is even). The fast path
// accepts v' when |v'| < 2^(kBits - 2) <= M/2; otherwise the tail compares
// against M/2 exactly and corrects by one M.
//
// X' - q' M is formed in 16-bit limbs: T_j = S_{2j} + 256 S_{2j+1} - q' M_j
// (|T_j| < 2^29), then one signed carry pass. The result is the limbs
// (16 bits each) and a final signed carry, which is 0 or -1 (the sign) for
// every accepted value.
//
// Everything here is constexpr (hence callable from host and device code
// alike), so the host checks build from this header with a plain C++ compiler.
#pragma once

#include <cstdint>

#include "tables.hpp"

namespace rns8x {

constexpr uint32_t kCrtFracBits = 14;

// Bit length of the product of the first P ladder moduli.
constexpr uint32_t ladder_bits(uint32_t P) {
  Limbs24 p;
  p.w[0] = 1;
  for (uint32_t i = 0; i < P; ++i) p.mul_add(kLadder[i], 0);
  uint32_t bits = 0;
  for (uint32_t l = 0; l < kWideLimbs; ++l)
    for (uint32_t b = 0; b < 24; ++b)
      if ((p.w[l] >> b) & 1u) bits = 24 * l + b + 1;
  return bits;
}

template <uint32_t P>
struct CrtTable {
  static constexpr uint32_t kBits = ladder_bits(P);
  // signed base-256 digits of any value below 2^kBits
  static constexpr uint32_t kDigits = (kBits + 1) / 8 + 1;
  static constexpr uint32_t kCols = kDigits + 2;  // + the two digits of F_i
  static constexpr uint32_t kLimbs = (kDigits + 1) / 2;  // 16-bit limbs of v
  static_assert(kCols <= 32, "one 32-column MFMA tile");
  // MFMA operand of lane l (column l & 31, planes 16 (l >> 5) .. +15), four
  // little-endian dwords of int8 weights w[plane][column]
  uint32_t frag[64][4];
  int8_t w[kMaxPrefix][32];
  uint32_t m16[kLimbs];    // M in 16-bit limbs
  uint32_t half16[kLimbs]; // M/2 in 16-bit limbs
};

template <uint32_t P>
constexpr CrtTable<P> make_crt_table() {
  using T = CrtTable<P>;
  T t{};
  Limbs24 prod;
  prod.w[0] = 1;
  for (uint32_t i = 0; i < P; ++i) prod.mul_add(kLadder[i], 0);
  double prod_d = 0.0, scale = 1.0;
  for (uint32_t l = 0; l < kWideLimbs; ++l, scale *= 16777216.0) prod_d += prod.w[l] * scale;
  for (uint32_t i = 0; i < P; ++i) {
    // K_i = (M / m_i) * ((M / m_i)^-1 mod m_i), below M
    Limbs24 k;
    k.w[0] = 1;
    for (uint32_t j = 0; j < P; ++j)
      if (j != i) k.mul_add(kLadder[j], 0);
    const uint32_t inv = P == 1 ? 1u : inverse_mod(k.mod_small(kLadder[i]), kLadder[i]);
    k.mul_add(inv, 0);
    // signed base-256 digits
    int carry = 0;
    for (uint32_t b = 0; b < T::kDigits; ++b) {
      const uint32_t byte = b / 3 < kWideLimbs ? (k.w[b / 3] >> (8 * (b % 3))) & 0xFFu : 0u;
      int v = static_cast<int>(byte) + carry;
      carry = v >= 128 ? 1 : 0;
      t.w[i][b] = static_cast<int8_t>(v - 256 * carry);
    }
    // F_i = round(2^kCrtFracBits K_i / M) in two signed digits
    double kd = 0.0;
    scale = 1.0;
    for (uint32_t l = 0; l < kWideLimbs; ++l, scale *= 16777216.0) kd += k.w[l] * scale;
    const int f = static_cast<int>(kd / prod_d * static_cast<double>(1u << kCrtFracBits) + 0.5);
    const int f0 = (f & 0xFF) >= 128 ? (f & 0xFF) - 256 : (f & 0xFF);
    t.w[i][T::kDigits] = static_cast<int8_t>(f0);
    t.w[i][T::kDigits + 1] = static_cast<int8_t>((f - f0) / 256);
  }
  for (uint32_t l = 0; l < 64; ++l)
    for (uint32_t q = 0; q < 4; ++q) {
      uint32_t word = 0;
      for (uint32_t b = 0; b < 4; ++b) {
        const uint32_t plane = 16 * (l >> 5) + 4 * q + b;
        const int8_t v = plane < P ? t.w[plane][l & 31] : int8_t{0};
        word |= static_cast<uint32_t>(static_cast<uint8_t>(v)) << (8 * b);
      }
      t.frag[l][q] = word;
    }
  // M and M/2 (M is even: m_0 = 256) in 16-bit limbs
  for (uint32_t j = 0; j < T::kLimbs; ++j) {
    uint32_t m = 0;
    for (uint32_t b = 0; b < 2; ++b) {
      const uint32_t byte_index = 2 * j + b;
      const uint32_t byte =
          byte_index / 3 < kWideLimbs ? (prod.w[byte_index / 3] >> (8 * (byte_index % 3))) & 0xFFu : 0u;
      m |= byte << (8 * b);
    }
    t.m16[j] = m;
  }
  for (uint32_t j = 0; j < T::kLimbs; ++j) {
    const uint32_t next = j + 1 < T::kLimbs ? t.m16[j + 1] : 0u;
    t.half16[j] = (t.m16[j] >> 1) | ((next & 1u) << 15);
  }
  return t;
}

// The centered value of one cell from its MFMA column sums S_b (b < kCols):
// 16-bit limbs of v (two's complement together with *sign, 0 or -1).
template <uint32_t P>
constexpr void crt_centered(const CrtTable<P>& t, const int32_t* s, uint32_t (&limb)[CrtTable<P>::kLimbs],
                            int32_t& sign) {
  using T = CrtTable<P>;
  const int32_t e = s[T::kDigits] + 256 * s[T::kDigits + 1];
  const int32_t q = (e + (1 << (kCrtFracBits - 1))) >> kCrtFracBits;
  int32_t c = 0;
#pragma unroll
  for (uint32_t j = 0; j < T::kLimbs; ++j) {
    const int32_t hi = 2 * j + 1 < T::kDigits ? s[2 * j + 1] : 0;
    const int32_t v = s[2 * j] + 256 * hi - q * static_cast<int32_t>(t.m16[j]) + c;
    limb[j] = static_cast<uint32_t>(v) & 0xFFFFu;
    c = v >> 16;
  }
  // fast path: |v'| < 2^(kBits - 2) <= M/2, so v' is the centered value
  constexpr uint32_t kT = T::kBits - 2;
  const int32_t sg = c >> 31;
  bool fast = c == sg;
#pragma unroll
  for (uint32_t j = kT / 16; j < T::kLimbs; ++j) {
    const uint32_t lo_bit = j == kT / 16 ? kT % 16 : 0u;
    fast &= (limb[j] >> lo_bit) == ((static_cast<uint32_t>(sg) & 0xFFFFu) >> lo_bit);
  }
  if (!fast) {
    // exact: v' + M/2 < 0 -> add M; v' - M/2 >= 0 -> subtract M
    uint32_t a[T::kLimbs] = {};
    int32_t ca = 0;
    for (uint32_t j = 0; j < T::kLimbs; ++j) {
      const int32_t v = static_cast<int32_t>(limb[j]) + static_cast<int32_t>(t.half16[j]) + ca;
      a[j] = static_cast<uint32_t>(v) & 0xFFFFu;
      ca = v >> 16;
    }
    ca += c;
    int32_t adj = 0;
    if (ca < 0) {
      adj = 1;
    } else {
      int32_t cb = 0;
      for (uint32_t j = 0; j < T::kLimbs; ++j) {
        const int32_t v = static_cast<int32_t>(a[j]) - static_cast<int32_t>(t.m16[j]) + cb;
        cb = v >> 16;
      }
      if (ca + cb >= 0) adj = -1;
    }
    int32_t cc = 0;
    for (uint32_t j = 0; j < T::kLimbs; ++j) {
      const int32_t v = static_cast<int32_t>(limb[j]) + adj * static_cast<int32_t>(t.m16[j]) + cc;
      limb[j] = static_cast<uint32_t>(v) & 0xFFFFu;
      cc = v >> 16;
    }
    c += cc;
  }
  sign = c;
}

// ---- 64-bit results (bounded int64 / uint64) at P = 9 .. 11 ------------------
//
// The same MFMA over the planes, with 14 weight columns per plane:
//   columns 0..7   signed base-256 digits of K_i mod 2^64, so
//                  X = sum_b 256^b S_b = X' (mod 2^64);
//   columns 8..13  signed base-256 digits of F_i = round(2^40 K_i / M), so
//                  E = sum_b 256^b S_{8+b} = 2^40 X'/M + err,
//                  |err| <= P * 128 * (1/2 + 2^-10) < kCrt64Err = 768
//                  (the table's F_i come from double quotients, which adds
//                  at most 2^-10 to each rounding error).
// With q = round(E / 2^40), the centered value is v = X' - q M whenever
// |v| < M/2 - (a few) and q is then exact, and g = E - 2^40 q =
// 2^40 v / M + err tells |v| apart from 2^63 and 2^64 (T63 = 2^103 / M,
// T64 = 2^104 / M in units of g) except within 3 * 1024 units, i.e. within
// 2^12 M / 2^40 of the edge. For P <= 11 (M < 2^87.1) that band is narrower
// than 2^62, and inside it the exact low 64 bits v mod 2^64 = X - q M
// (mod 2^64) decide: a value near +2^63 is below 2^63 iff its low word, read
// as int64, is non-negative; near -2^63 at or above -2^63 iff it is
// negative; near 2^64 below 2^64 iff the low word is at least 2^63. If q is
// off by one (|v| near M/2, far out of every 64-bit range), |g| is near
// 2^39 and the value is refused. The decisions use g8 = floor(g / 256) in
// 32 bits; the thresholds below carry that loss.
constexpr uint32_t kCrt64Cols = 14;
constexpr uint32_t kCrt64FracBits = 40;
constexpr int32_t kCrt64Err = 768;
constexpr uint32_t kCrt64MinP = 9, kCrt64MaxP = 11;

template <uint32_t P>
struct Crt64Table {
  static_assert(P >= kCrt64MinP && P <= kCrt64MaxP, "the 64-bit CRT tail covers prefixes 9..11");
  uint32_t frag[64][4];  // MFMA operand, same layout as CrtTable::frag
  int8_t w[kMaxPrefix][32];
  uint64_t m64;          // M mod 2^64
  // g8 thresholds: |g8| <= in63 -> |v| < 2^63; |g8| >= out63 -> |v| > 2^63;
  // in between the low word decides. Likewise in64 / out64 for 2^64 and
  // small: |g8| <= small -> |v| < 2^62, g8 < -small -> v < 0.
  int32_t in63, out63, in64, out64, small;
};

template <uint32_t P>
constexpr Crt64Table<P> make_crt64_table() {
  using T = Crt64Table<P>;
  T t{};
  Limbs24 prod;
  prod.w[0] = 1;
  for (uint32_t i = 0; i < P; ++i) prod.mul_add(kLadder[i], 0);
  double prod_d = 0.0, scale = 1.0;
  for (uint32_t l = 0; l < kWideLimbs; ++l, scale *= 16777216.0) prod_d += prod.w[l] * scale;
  auto low64 = [](const Limbs24& x) {
    uint64_t v = 0;
    for (uint32_t l = 0; l < 3; ++l) v |= static_cast<uint64_t>(x.w[l]) << (24 * l);  // bits 48..71 wrap away
    return v;
  };
  for (uint32_t i = 0; i < P; ++i) {
    Limbs24 k;
    k.w[0] = 1;
    for (uint32_t j = 0; j < P; ++j)
      if (j != i) k.mul_add(kLadder[j], 0);
    const uint32_t inv = inverse_mod(k.mod_small(kLadder[i]), kLadder[i]);
    k.mul_add(inv, 0);
    // K_i mod 2^64 in 8 signed digits (the carry out of the top digit is a
    // multiple of 2^64)
    const uint64_t k64 = low64(k);
    int carry = 0;
    for (uint32_t b = 0; b < 8; ++b) {
      const int v = static_cast<int>((k64 >> (8 * b)) & 0xFFu) + carry;
      carry = v >= 128 ? 1 : 0;
      t.w[i][b] = static_cast<int8_t>(v - 256 * carry);
    }
    double kd = 0.0;
    scale = 1.0;
    for (uint32_t l = 0; l < kWideLimbs; ++l, scale *= 16777216.0) kd += k.w[l] * scale;
    const int64_t f = static_cast<int64_t>(kd / prod_d * 1099511627776.0 + 0.5);  // 2^40 K_i / M, rounded
    carry = 0;
    for (uint32_t b = 0; b < 6; ++b) {
      const int v = static_cast<int>((f >> (8 * b)) & 0xFF) + carry;
      carry = v >= 128 ? 1 : 0;
      t.w[i][8 + b] = static_cast<int8_t>(v - 256 * carry);
    }
  }
  for (uint32_t l = 0; l < 64; ++l)
    for (uint32_t q = 0; q < 4; ++q) {
      uint32_t word = 0;
      for (uint32_t b = 0; b < 4; ++b) {
        const uint32_t plane = 16 * (l >> 5) + 4 * q + b;
        const int8_t v = plane < P ? t.w[plane][l & 31] : int8_t{0};
        word |= static_cast<uint32_t>(static_cast<uint8_t>(v)) << (8 * b);
      }
      t.frag[l][q] = word;
    }
  t.m64 = low64(prod);
  // thresholds in units of 256 of g, with the rounding error and the floor of
  // g8 on the safe side (two units of margin for the double quotients)
  const double t63 = 10141204801825835211973625643008.0 / prod_d;   // 2^103 / M
  const double t64 = 20282409603651670423947251286016.0 / prod_d;   // 2^104 / M
  t.in63 = static_cast<int32_t>((t63 - kCrt64Err) / 256.0) - 2;
  t.out63 = static_cast<int32_t>((t63 + kCrt64Err) / 256.0) + 3;
  t.in64 = static_cast<int32_t>((t64 - kCrt64Err) / 256.0) - 2;
  t.out64 = static_cast<int32_t>((t64 + kCrt64Err) / 256.0) + 3;
  t.small = kCrt64Err / 256 + 2;
  return t;
}

// One cell's column sums s[0..13] -> the low 64 bits of v = X' - q M and
// g8 = floor((E - 2^40 q) / 256). Every step is a 32-bit operation except
// the one 32 x 32 -> 64-bit multiply-add by M mod 2^64 (|S_b| < 2^18, so the
// pair sums below fit 27 bits):
//   floor(E / 2^32) = e45 + ((e23 + (e01 >> 16)) >> 16)   (arithmetic shifts
//       are floors, and floor(floor(x / a) / b) = floor(x / ab));
//   q = floor((E + 2^39) / 2^40) = (floor(E / 2^32) + 2^7) >> 8;
//   g8 = floor(E / 256) - 2^32 q lies in [-2^31, 2^31), so it is the low
//       word of floor(E / 256) = e45 2^24 + e23 2^8 + (e01 >> 8);
//   X mod 2^64: low word x01 + (x23 << 16), high word
//       ((x23 + (x01 >> 16)) >> 16) + x45 + (x67 << 16), by the same floors.
template <uint32_t P>
constexpr uint64_t crt64_low(const Crt64Table<P>& t, const int32_t* s, int32_t& g8) {
  const int32_t e01 = s[8] + s[9] * 256, e23 = s[10] + s[11] * 256, e45 = s[12] + s[13] * 256;
  const int32_t e32 = e45 + ((e23 + (e01 >> 16)) >> 16);
  const int32_t q = (e32 + 128) >> 8;
  g8 = static_cast<int32_t>(static_cast<uint32_t>(e01 >> 8) + (static_cast<uint32_t>(e23) << 8) +
                            (static_cast<uint32_t>(e45) << 24));
  const int32_t x01 = s[0] + s[1] * 256, x23 = s[2] + s[3] * 256, x45 = s[4] + s[5] * 256, x67 = s[6] + s[7] * 256;
  const uint32_t xlo = static_cast<uint32_t>(x01) + (static_cast<uint32_t>(x23) << 16);
  const uint32_t xhi = static_cast<uint32_t>((x23 + (x01 >> 16)) >> 16) + static_cast<uint32_t>(x45) +
                       (static_cast<uint32_t>(x67) << 16);
  const uint64_t x = (static_cast<uint64_t>(xhi) << 32) | xlo;
  return x - static_cast<uint64_t>(static_cast<int64_t>(q)) * t.m64;
}

// Whether v (low word lo, class g8) lies in int64: [-2^63, 2^63).
template <uint32_t P>
constexpr bool crt64_in_int64(const Crt64Table<P>& t, uint64_t lo, int32_t g8) {
  // |g8| as uint32 (g8 = -2^31 when g = -2^39); branch-free
  const uint32_t a = g8 < 0 ? 0u - static_cast<uint32_t>(g8) : static_cast<uint32_t>(g8);
  const bool inside = a <= static_cast<uint32_t>(t.in63);
  const bool outside = a >= static_cast<uint32_t>(t.out63);
  const bool band = (static_cast<int32_t>(lo >> 32) < 0) == (g8 < 0);
  return inside | (!outside & band);
}

// Whether v lies in [0, 2^64) (then the canonical value is lo).
template <uint32_t P>
constexpr bool crt64_in_uint64(const Crt64Table<P>& t, uint64_t lo, int32_t g8) {
  // branch-free: (g8 in [-small, small] and lo >= 0 as int64) or
  // (g8 in (small, in64]) or (g8 in (in64, out64) and lo >= 2^63)
  const bool neg_lo = static_cast<int32_t>(lo >> 32) < 0;
  const bool small = (g8 >= -t.small) & (g8 <= t.small);
  const bool mid = (g8 > t.small) & (g8 <= t.in64);
  const bool band = (g8 > t.in64) & (g8 < t.out64);
  return (small & !neg_lo) | mid | (band & neg_lo);
}

// Whether crt_export_kernel can address an export: it computes plane offsets
// from the first plane (plane_span bytes up to the end of the last plane's
// rows), an output row's byte range (n * 8 * limbs) and a lane's offset in
// it in 32 bits, and numbers its (row, 64-column chunk) units in 32 bits.
// Exports outside these limits run the Garner kernel, which uses 64-bit
// offsets.
constexpr bool crt_export_fits(uint64_t plane_span, int64_t m, int64_t n, uint32_t limbs) {
  if (m <= 0 || n <= 0 || limbs == 0) return false;
  if (plane_span >= (uint64_t{1} << 31)) return false;
  if (static_cast<uint64_t>(n) * 8u * limbs >= (uint64_t{1} << 31)) return false;
  return static_cast<uint64_t>(m) * ((static_cast<uint64_t>(n) + 63u) / 64u) < (uint64_t{1} << 32);
}

}  // namespace rns8x
