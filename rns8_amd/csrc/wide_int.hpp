// Fixed-width 256-bit two's-complement integers for host-side contract math.
//
// The reference performs prefix selection, CRT range checks and exact-wide
// magnitude proofs with Boost cpp_int (src/core/moduli.cpp, exact_range.hpp).
// Every quantity on this path is bounded well below 2^192 (modulus products
// < 2^155, K * 2^128 < 2^159, sums of 2^31 values below 2^64 < 2^95, and the
// products formed in the exact-wide bound < 2^192), so 256 bits represent
// them exactly. Division is only ever by 2 (axis midpoints) and truncates
// toward zero like cpp_int.
#pragma once

#include <cstdint>

namespace rns8x {

struct I256 {
  uint64_t w[4] = {0, 0, 0, 0};

  static I256 from_u64(uint64_t v) {
    I256 r;
    r.w[0] = v;
    return r;
  }
  static I256 from_i64(int64_t v) {
    I256 r;
    r.w[0] = static_cast<uint64_t>(v);
    const uint64_t fill = v < 0 ? ~uint64_t{0} : 0;
    r.w[1] = r.w[2] = r.w[3] = fill;
    return r;
  }
  static I256 pow2(unsigned bits) {
    I256 r;
    if (bits < 256) r.w[bits / 64] = uint64_t{1} << (bits % 64);
    return r;
  }
  bool negative() const { return (w[3] >> 63) != 0; }
  bool is_zero() const { return (w[0] | w[1] | w[2] | w[3]) == 0; }

  friend I256 operator+(const I256& a, const I256& b) {
    I256 r;
    unsigned __int128 c = 0;
    for (int i = 0; i < 4; ++i) {
      c += static_cast<unsigned __int128>(a.w[i]) + b.w[i];
      r.w[i] = static_cast<uint64_t>(c);
      c >>= 64;
    }
    return r;
  }
  I256 operator-() const {
    I256 r;
    for (int i = 0; i < 4; ++i) r.w[i] = ~w[i];
    return r + from_u64(1);
  }
  friend I256 operator-(const I256& a, const I256& b) { return a + (-b); }
  // product modulo 2^256 (exact for every operand range used here)
  friend I256 operator*(const I256& a, const I256& b) {
    I256 r;
    for (int i = 0; i < 4; ++i) {
      unsigned __int128 carry = 0;
      for (int j = 0; i + j < 4; ++j) {
        const unsigned __int128 t = static_cast<unsigned __int128>(a.w[i]) * b.w[j] + r.w[i + j] + carry;
        r.w[i + j] = static_cast<uint64_t>(t);
        carry = t >> 64;
      }
    }
    return r;
  }
  friend bool operator<(const I256& a, const I256& b) {
    if (a.negative() != b.negative()) return a.negative();
    for (int i = 3; i >= 0; --i)
      if (a.w[i] != b.w[i]) return a.w[i] < b.w[i];
    return false;
  }
  friend bool operator>(const I256& a, const I256& b) { return b < a; }
  friend bool operator<=(const I256& a, const I256& b) { return !(b < a); }
  friend bool operator>=(const I256& a, const I256& b) { return !(a < b); }
  friend bool operator==(const I256& a, const I256& b) {
    return a.w[0] == b.w[0] && a.w[1] == b.w[1] && a.w[2] == b.w[2] && a.w[3] == b.w[3];
  }
  friend bool operator!=(const I256& a, const I256& b) { return !(a == b); }

  I256 abs() const { return negative() ? -*this : *this; }
  // truncating division by 2 (toward zero), matching C++/cpp_int semantics
  I256 half_trunc() const {
    const bool neg = negative();
    I256 m = neg ? -*this : *this;
    for (int i = 0; i < 4; ++i) m.w[i] = (m.w[i] >> 1) | (i < 3 ? (m.w[i + 1] << 63) : 0);
    return neg ? -m : m;
  }
  uint32_t bit_length() const {  // of a non-negative value
    for (int i = 3; i >= 0; --i) {
      if (w[i]) return static_cast<uint32_t>(64 * i + 64 - __builtin_clzll(w[i]));
    }
    return 0;
  }
  bool fits_u64() const { return !negative() && (w[1] | w[2] | w[3]) == 0; }
};

inline I256 imin(const I256& a, const I256& b) { return b < a ? b : a; }
inline I256 imax(const I256& a, const I256& b) { return a < b ? b : a; }

}  // namespace rns8x
