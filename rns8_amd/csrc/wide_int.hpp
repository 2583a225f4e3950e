// Fixed-width two's-complement integers for host-side contract math.
//
// The reference performs prefix selection, CRT range checks and exact-wide
// magnitude proofs with Boost cpp_int (src/core/moduli.cpp, exact_range.hpp).
// Here they use fixed widths chosen so that no quantity can wrap:
//   * I256 (4 limbs): prefix selection and plan-level range checks. Modulus
//     products are below 2^155, K * 2^128 below 2^191, 2 * bound below 2^65.
//   * I512 (8 limbs): exact-wide admission (exact_range.hpp). A carried
//     operand summary comes from an admitted GEMM, so its largest magnitude
//     is below P/2 < 2^155 and its absolute sums below 2^63 * 2^155 = 2^218;
//     native operands are below 2^64 with sums below 2^127. Every candidate
//     product of the cell bound (K * max * max, abs_sum * max, centre * sum,
//     K * centre * centre, K * dev * dev, dev_sum * dev) is therefore below
//     2^63 * 2^155 * 2^155 = 2^373, a cell bound before the range decision is
//     at most that, and a row or column sum of 2^63 such bounds stays below
//     2^437, well inside 511 bits.
// Division is only ever by 2 (axis midpoints) and truncates toward zero like
// cpp_int.
#pragma once

#include <cstdint>

namespace rns8x {

template <int L>
struct WideInt {
  static_assert(L >= 2, "at least 128 bits");
  uint64_t w[L] = {};

  static WideInt from_u64(uint64_t v) {
    WideInt r;
    r.w[0] = v;
    return r;
  }
  static WideInt from_i64(int64_t v) {
    WideInt r;
    r.w[0] = static_cast<uint64_t>(v);
    const uint64_t fill = v < 0 ? ~uint64_t{0} : 0;
    for (int i = 1; i < L; ++i) r.w[i] = fill;
    return r;
  }
  static WideInt pow2(unsigned bits) {
    WideInt r;
    if (bits < 64u * L) r.w[bits / 64] = uint64_t{1} << (bits % 64);
    return r;
  }
  // sign-extending conversion from a narrower (or equal) width
  template <int M>
  static WideInt widen(const WideInt<M>& v) {
    static_assert(M <= L, "widen only");
    WideInt r;
    for (int i = 0; i < M; ++i) r.w[i] = v.w[i];
    const uint64_t fill = v.negative() ? ~uint64_t{0} : 0;
    for (int i = M; i < L; ++i) r.w[i] = fill;
    return r;
  }
  bool negative() const { return (w[L - 1] >> 63) != 0; }
  bool is_zero() const {
    uint64_t o = 0;
    for (int i = 0; i < L; ++i) o |= w[i];
    return o == 0;
  }

  friend WideInt operator+(const WideInt& a, const WideInt& b) {
    WideInt r;
    unsigned __int128 c = 0;
    for (int i = 0; i < L; ++i) {
      c += static_cast<unsigned __int128>(a.w[i]) + b.w[i];
      r.w[i] = static_cast<uint64_t>(c);
      c >>= 64;
    }
    return r;
  }
  WideInt operator-() const {
    WideInt r;
    for (int i = 0; i < L; ++i) r.w[i] = ~w[i];
    return r + from_u64(1);
  }
  friend WideInt operator-(const WideInt& a, const WideInt& b) { return a + (-b); }
  // number of limbs up to the highest nonzero one (of a non-negative value)
  int used_limbs() const {
    for (int i = L - 1; i >= 0; --i)
      if (w[i]) return i + 1;
    return 0;
  }
  // Product modulo 2^(64 L). Schoolbook over the magnitudes' used limbs, so
  // the small values that dominate the proofs cost a few limb products; the
  // sign is applied afterwards (two's complement product mod 2^(64 L)).
  friend WideInt operator*(const WideInt& a, const WideInt& b) {
    const bool neg = a.negative() != b.negative();
    const WideInt x = a.abs(), y = b.abs();
    const int nx = x.used_limbs(), ny = y.used_limbs();
    WideInt r;
    for (int i = 0; i < nx; ++i) {
      unsigned __int128 carry = 0;
      int j = 0;
      for (; j < ny && i + j < L; ++j) {
        const unsigned __int128 t = static_cast<unsigned __int128>(x.w[i]) * y.w[j] + r.w[i + j] + carry;
        r.w[i + j] = static_cast<uint64_t>(t);
        carry = t >> 64;
      }
      if (i + j < L) r.w[i + j] = static_cast<uint64_t>(carry);
    }
    return neg ? -r : r;
  }
  friend bool operator<(const WideInt& a, const WideInt& b) {
    if (a.negative() != b.negative()) return a.negative();
    for (int i = L - 1; i >= 0; --i)
      if (a.w[i] != b.w[i]) return a.w[i] < b.w[i];
    return false;
  }
  friend bool operator>(const WideInt& a, const WideInt& b) { return b < a; }
  friend bool operator<=(const WideInt& a, const WideInt& b) { return !(b < a); }
  friend bool operator>=(const WideInt& a, const WideInt& b) { return !(a < b); }
  friend bool operator==(const WideInt& a, const WideInt& b) {
    for (int i = 0; i < L; ++i)
      if (a.w[i] != b.w[i]) return false;
    return true;
  }
  friend bool operator!=(const WideInt& a, const WideInt& b) { return !(a == b); }

  WideInt abs() const { return negative() ? -*this : *this; }
  // truncating division by 2 (toward zero), matching C++/cpp_int semantics
  WideInt half_trunc() const {
    const bool neg = negative();
    WideInt m = neg ? -*this : *this;
    for (int i = 0; i < L; ++i) m.w[i] = (m.w[i] >> 1) | (i < L - 1 ? (m.w[i + 1] << 63) : 0);
    return neg ? -m : m;
  }
  uint32_t bit_length() const {  // of a non-negative value
    for (int i = L - 1; i >= 0; --i) {
      if (w[i]) return static_cast<uint32_t>(64 * i + 64 - __builtin_clzll(w[i]));
    }
    return 0;
  }
  bool fits_u64() const {
    if (negative()) return false;
    for (int i = 1; i < L; ++i)
      if (w[i]) return false;
    return true;
  }
};

template <int L>
inline WideInt<L> imin(const WideInt<L>& a, const WideInt<L>& b) {
  return b < a ? b : a;
}
template <int L>
inline WideInt<L> imax(const WideInt<L>& a, const WideInt<L>& b) {
  return a < b ? b : a;
}

using I256 = WideInt<4>;
using I512 = WideInt<8>;

}  // namespace rns8x
