// Exact-wide magnitude proofs in fixed-width integers, for the device
// kernels (exact_axes.hip) and the host alike (reference
// src/core/exact_range.hpp:16-157).
//
// A packed exact-wide operand carries, per row and per column, the
// reference's axis summary (max |x|, sum |x|, sum x, min x, max x, and the
// sum of |x - centre|); a GEMM result carries per-row and per-column maxima
// and sums of its cell bounds. The cell bound of C = A x B at (r, c) is the
// minimum of the reference's candidates built from A's row r and B's column
// c, and C's bound is min(k * maxA * maxB, max over cells).
//
// Widths. A native (64-bit) operand's summaries fit 128 bits: k < 2^63
// values of magnitude <= 2^64 sum below 2^127, and every centre, deviation
// and maximum is below 2^64. Every candidate of two native axes is then a
// product of a 128-bit and a 64-bit factor (below 2^192), and the centre term
// is below 2^194: 256-bit arithmetic is exact for them. Carried summaries
// (of earlier results) can make candidates exceed 2^256, so products and sums
// that involve them saturate at 2^256 - 1. Saturation is monotone and
// commutes with min, max, + and x on non-negative integers
// (sat(sat(a) x b) = sat(a x b), likewise for +), so every saturated
// quantity equals sat(the unbounded one), and every admission decision,
// which compares against a modulus product below 2^160, equals the unbounded
// decision. A product that is admitted has every cell below 2^160, so the
// summaries it carries are exact.
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define RNS8_XA __host__ __device__ inline
#else
#define RNS8_XA inline
#endif

namespace rns8x {
namespace xa {

using u64 = uint64_t;
using u128 = unsigned __int128;
using i128 = __int128;

// Unsigned 256-bit integer, little-endian 64-bit words. Also holds 256-bit
// two's complement values where stated.
struct U256 {
  u64 w[4];
};

RNS8_XA U256 zero256() { return U256{{0, 0, 0, 0}}; }
RNS8_XA U256 sat256() { return U256{{~u64{0}, ~u64{0}, ~u64{0}, ~u64{0}}}; }
RNS8_XA U256 from128(u128 v) { return U256{{static_cast<u64>(v), static_cast<u64>(v >> 64), 0, 0}}; }

RNS8_XA bool less(const U256& a, const U256& b) {
  if (a.w[3] != b.w[3]) return a.w[3] < b.w[3];
  if (a.w[2] != b.w[2]) return a.w[2] < b.w[2];
  if (a.w[1] != b.w[1]) return a.w[1] < b.w[1];
  return a.w[0] < b.w[0];
}
RNS8_XA U256 min256(const U256& a, const U256& b) { return less(b, a) ? b : a; }
RNS8_XA U256 max256(const U256& a, const U256& b) { return less(a, b) ? b : a; }
RNS8_XA bool is_zero(const U256& a) { return (a.w[0] | a.w[1] | a.w[2] | a.w[3]) == 0; }

// a + b mod 2^256; *carry receives the bit shifted out
RNS8_XA U256 add256(const U256& a, const U256& b, u64* carry) {
  U256 r;
  u64 c = 0;
  for (int i = 0; i < 4; ++i) {
    const u128 t = static_cast<u128>(a.w[i]) + b.w[i] + c;
    r.w[i] = static_cast<u64>(t);
    c = static_cast<u64>(t >> 64);
  }
  *carry = c;
  return r;
}
RNS8_XA U256 sat_add(const U256& a, const U256& b) {
  u64 c;
  const U256 r = add256(a, b, &c);
  return c ? sat256() : r;
}
// a - b mod 2^256
RNS8_XA U256 sub256(const U256& a, const U256& b) {
  U256 r;
  u64 borrow = 0;
  for (int i = 0; i < 4; ++i) {
    const u128 t = static_cast<u128>(a.w[i]) - b.w[i] - borrow;
    r.w[i] = static_cast<u64>(t);
    borrow = static_cast<u64>(t >> 64) & 1u;
  }
  return r;
}
RNS8_XA bool negative256(const U256& a) { return (a.w[3] >> 63) != 0; }
RNS8_XA U256 abs256(const U256& a) { return negative256(a) ? sub256(zero256(), a) : a; }

// a * b for a < 2^128, b < 2^64: exact (below 2^192)
RNS8_XA U256 mul_128_64(u128 a, u64 b) {
  const u128 lo = static_cast<u128>(static_cast<u64>(a)) * b;
  const u128 hi = static_cast<u128>(static_cast<u64>(a >> 64)) * b + (lo >> 64);
  return U256{{static_cast<u64>(lo), static_cast<u64>(hi), static_cast<u64>(hi >> 64), 0}};
}
// signed a * b for |a| < 2^127, |b| < 2^64, as 256-bit two's complement
RNS8_XA U256 smul_128_64(i128 a, i128 b) {
  const bool neg = (a < 0) != (b < 0);
  const u128 ma = static_cast<u128>(a < 0 ? -a : a);
  const u64 mb = static_cast<u64>(b < 0 ? -b : b);
  const U256 p = mul_128_64(ma, mb);
  return neg ? sub256(zero256(), p) : p;
}

// min(a * b, 2^256 - 1): the schoolbook product in eight words, with
// compile-time indices only (registers, no local memory)
RNS8_XA U256 sat_mul(const U256& a, const U256& b) {
  u64 r[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    u64 c = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u128 t = static_cast<u128>(a.w[i]) * b.w[j] + r[i + j] + c;
      r[i + j] = static_cast<u64>(t);
      c = static_cast<u64>(t >> 64);
    }
    r[i + 4] = c;
  }
  if ((r[4] | r[5] | r[6] | r[7]) != 0) return sat256();
  return U256{{r[0], r[1], r[2], r[3]}};
}
RNS8_XA U256 sat_mul64(u64 a, const U256& b) { return sat_mul(U256{{a, 0, 0, 0}}, b); }

// ---- axis summaries ----------------------------------------------------------

// One row or column of a proof, as it lies in device memory (128 bytes,
// little-endian words; the layout of rns8_mi355x_exact_axis). Native axes
// fill every field; carried axes (of GEMM results) only the first two.
struct alignas(16) AxisRecord {
  u64 max_magnitude[4];  // unsigned 256-bit
  u64 absolute_sum[4];   // unsigned 256-bit
  u64 sum[2];            // signed 128-bit
  u64 minimum[2];        // signed 128-bit
  u64 maximum[2];        // signed 128-bit
  u64 deviation_sum[2];  // unsigned 128-bit
};
static_assert(sizeof(AxisRecord) == 128, "record layout");

// What an operand's axes are: native summaries (of a pack), carried maxima
// and sums (of a GEMM result), or none, when every axis is the uniform one
// derived from the operand's global maximum (exact_range.hpp:101-106).
enum class AxisKind : uint32_t { Native = 0, Carried = 1, Uniform = 2 };

RNS8_XA i128 get_i128(const u64* w) { return static_cast<i128>((static_cast<u128>(w[1]) << 64) | w[0]); }
RNS8_XA u128 get_u128(const u64* w) { return (static_cast<u128>(w[1]) << 64) | w[0]; }
RNS8_XA void put_u128(u64* w, u128 v) {
  w[0] = static_cast<u64>(v);
  w[1] = static_cast<u64>(v >> 64);
}
RNS8_XA U256 get_u256(const u64* w) { return U256{{w[0], w[1], w[2], w[3]}}; }
RNS8_XA void put_u256(u64* w, const U256& v) {
  for (int i = 0; i < 4; ++i) w[i] = v.w[i];
}

// (min + max) / 2 truncated toward zero, as the reference's integer
// division does (exact_range.hpp:24-26)
RNS8_XA i128 axis_centre(i128 lo, i128 hi) {
  const i128 s = lo + hi;
  return (s + (s < 0 ? 1 : 0)) >> 1;
}

// The factors of an axis that the cell bounds use, computed once per axis
// (exact_range.hpp:80-99 with k folded in where it multiplies one axis).
struct AxisTerms {
  bool native;
  u64 k;
  // every kind
  U256 max_magnitude, absolute_sum;
  // native axes only (widths in the header comment)
  u64 max64;
  u128 abs128, k_max128, dev_sum, k_dev;
  u64 dev;
  i128 sum, centre, k_centre;
};

// r: the axis's record (not read for a uniform axis)
RNS8_XA AxisTerms axis_terms(const AxisRecord* r, AxisKind kind, const U256& global_max, u64 k) {
  AxisTerms t{};
  t.native = kind == AxisKind::Native;
  t.k = k;
  if (kind == AxisKind::Uniform) {
    t.max_magnitude = global_max;
    t.absolute_sum = sat_mul64(k, global_max);
  } else {
    t.max_magnitude = get_u256(r->max_magnitude);
    t.absolute_sum = get_u256(r->absolute_sum);
  }
  if (t.native) {
    t.max64 = r->max_magnitude[0];
    t.abs128 = get_u128(r->absolute_sum);
    t.k_max128 = static_cast<u128>(k) * t.max64;
    t.sum = get_i128(r->sum);
    const i128 lo = get_i128(r->minimum), hi = get_i128(r->maximum);
    t.centre = axis_centre(lo, hi);
    const i128 dl = lo - t.centre, dh = hi - t.centre;
    const u128 ml = static_cast<u128>(dl < 0 ? -dl : dl), mh = static_cast<u128>(dh < 0 ? -dh : dh);
    t.dev = static_cast<u64>(ml > mh ? ml : mh);
    t.dev_sum = get_u128(r->deviation_sum);
    t.k_dev = static_cast<u128>(k) * t.dev;
    t.k_centre = static_cast<i128>(k) * t.centre;
  }
  return t;
}

// Bound on |dot(row a, column b)| (exact_range.hpp:80-99): the minimum of
// k maxA maxB, |a|_1 maxB, maxA |b|_1 and, for two native axes,
// |cA sum(b) + cB sum(a) - k cA cB| + min(k dA dB, devsumA dB, dA devsumB).
RNS8_XA U256 cell_bound(const AxisTerms& a, const AxisTerms& b) {
  if (a.native && b.native) {
    U256 bound = mul_128_64(a.k_max128, b.max64);
    bound = min256(bound, mul_128_64(a.abs128, b.max64));
    bound = min256(bound, mul_128_64(b.abs128, a.max64));
    U256 rem = mul_128_64(a.k_dev, b.dev);
    rem = min256(rem, mul_128_64(a.dev_sum, b.dev));
    rem = min256(rem, mul_128_64(b.dev_sum, a.dev));
    // cA sum(b) + cB sum(a) - (k cA) cB, below 2^194 in magnitude
    u64 c;
    const U256 t = sub256(add256(smul_128_64(b.sum, a.centre), smul_128_64(a.sum, b.centre), &c),
                          smul_128_64(a.k_centre, b.centre));
    return min256(bound, add256(abs256(t), rem, &c));
  }
  U256 bound = sat_mul(sat_mul64(a.k, a.max_magnitude), b.max_magnitude);
  bound = min256(bound, sat_mul(a.absolute_sum, b.max_magnitude));
  return min256(bound, sat_mul(a.max_magnitude, b.absolute_sum));
}

// ---- native summaries: what the pack-time passes compute ------------------

// A partial summary of part of one axis (one 64 x 64 tile's share of a row
// or a column), in "biased" values u (x + 2^63 for int64, x for uint64),
// whose unsigned order is the order of x. Pass 1 fills every field; pass 2
// keeps the sum of |x - centre| in `sum`. Partials of at most 2^63 values
// are exact in these widths (sums below 2^127).
struct alignas(16) AxisPartial {
  u64 hi;      // max u
  u64 not_lo;  // max ~u, that is ~(min u)
  u128 sum;    // sum of u (pass 2: sum of |x - centre|)
  u128 abs_sum;
};
static_assert(sizeof(AxisPartial) == 48, "partial layout");

RNS8_XA u64 bias(u64 raw, bool is_signed) { return is_signed ? raw ^ (u64{1} << 63) : raw; }
RNS8_XA i128 unbias(u64 u, bool is_signed) {
  return is_signed ? static_cast<i128>(static_cast<int64_t>(u ^ (u64{1} << 63))) : static_cast<i128>(u);
}
RNS8_XA u64 magnitude(u64 raw, bool is_signed) {
  if (!is_signed) return raw;
  const int64_t x = static_cast<int64_t>(raw);
  return x < 0 ? u64{0} - raw : raw;  // |INT64_MIN| = 2^63 fits
}
RNS8_XA AxisPartial empty_partial() { return AxisPartial{0, 0, 0, 0}; }
RNS8_XA void partial_add(AxisPartial& p, u64 raw, bool is_signed) {
  const u64 u = bias(raw, is_signed);
  p.hi = u > p.hi ? u : p.hi;
  p.not_lo = ~u > p.not_lo ? ~u : p.not_lo;
  p.sum += u;
  p.abs_sum += magnitude(raw, is_signed);
}
RNS8_XA void partial_merge(AxisPartial& p, const AxisPartial& o) {
  p.hi = o.hi > p.hi ? o.hi : p.hi;
  p.not_lo = o.not_lo > p.not_lo ? o.not_lo : p.not_lo;
  p.sum += o.sum;
  p.abs_sum += o.abs_sum;
}
// The running partial of one lane over at most 2^32 values, with the sums
// as a 64-bit word plus a count of carries out of it.
struct PartialAcc {
  u64 hi = 0, not_lo = 0, sum = 0, abs_sum = 0;
  uint32_t sum_carries = 0, abs_carries = 0;
  RNS8_XA void add(u64 raw, bool is_signed) {
    const u64 u = bias(raw, is_signed), mag = magnitude(raw, is_signed);
    hi = u > hi ? u : hi;
    not_lo = ~u > not_lo ? ~u : not_lo;
    sum += u;
    sum_carries += sum < u ? 1u : 0u;
    abs_sum += mag;
    abs_carries += abs_sum < mag ? 1u : 0u;
  }
  RNS8_XA AxisPartial partial() const {
    return AxisPartial{hi, not_lo, (static_cast<u128>(sum_carries) << 64) | sum,
                       (static_cast<u128>(abs_carries) << 64) | abs_sum};
  }
};
// the same for pass 2's deviation sums
struct DeviationAcc {
  u64 sum = 0;
  uint32_t carries = 0;
  RNS8_XA void add(u64 d) {
    sum += d;
    carries += sum < d ? 1u : 0u;
  }
  RNS8_XA u128 value() const { return (static_cast<u128>(carries) << 64) | sum; }
};

// |x - centre| for pass 2 (below 2^64: centre lies between the extremes)
RNS8_XA u64 deviation(u64 raw, i128 centre, bool is_signed) {
  const i128 d = unbias(bias(raw, is_signed), is_signed) - centre;
  return static_cast<u64>(d < 0 ? -d : d);
}
RNS8_XA i128 record_centre(const AxisRecord& r) { return axis_centre(get_i128(r.minimum), get_i128(r.maximum)); }

// The record of a native axis of `count` values from its merged pass-1
// partial (the deviation sum is added by pass 2).
RNS8_XA AxisRecord native_record(const AxisPartial& p, u64 count, bool is_signed) {
  AxisRecord r{};
  const i128 lo = unbias(~p.not_lo, is_signed), hi = unbias(p.hi, is_signed);
  const u128 mlo = static_cast<u128>(lo < 0 ? -lo : lo), mhi = static_cast<u128>(hi < 0 ? -hi : hi);
  put_u256(r.max_magnitude, from128(mlo > mhi ? mlo : mhi));
  put_u256(r.absolute_sum, from128(p.abs_sum));
  const i128 sum = is_signed ? static_cast<i128>(p.sum) - (static_cast<i128>(count) << 63) : static_cast<i128>(p.sum);
  put_u128(r.sum, static_cast<u128>(sum));
  put_u128(r.minimum, static_cast<u128>(lo));
  put_u128(r.maximum, static_cast<u128>(hi));
  return r;
}

}  // namespace xa
}  // namespace rns8x
