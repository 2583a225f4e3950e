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
