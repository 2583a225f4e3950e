// Exact-wide magnitude proofs (reference src/core/exact_range.hpp:16-171),
// host C++ over 512-bit integers.
//
// A packed exact-wide operand carries its largest magnitude and, when it came
// from host memory or from an earlier GEMM, per-row and per-column summaries.
// A GEMM C = A x B is admitted iff the bound it proves for |C| fits the
// prefix's CRT range (2 * bound < P signed, bound < P unsigned); C then
// carries that bound and its own row and column summaries into later GEMMs.
// The reference computes these with unbounded integers; the widths here are
// sized so that nothing wraps (wide_int.hpp states the limits), which makes
// every decision equal to the unbounded one.
#pragma once

#include <algorithm>
#include <cstdint>
#include <thread>
#include <type_traits>
#include <vector>

#include "rns8/rns8.h"
#include "shards.hpp"
#include "wide_int.hpp"

// Exact-wide per-axis magnitude summary (reference src/core/internal.hpp:72-86
// rns8_exact_axis_range): used to tighten the output bound of a GEMM.
struct ExactAxis {
  rns8x::I512 max_magnitude;
  rns8x::I512 absolute_sum;
  rns8x::I512 sum;
  rns8x::I512 minimum;
  rns8x::I512 maximum;
  rns8x::I512 deviation_sum;
  bool sum_known = false;
};

namespace rns8x {

// exact_range.hpp:16-18
inline bool exact_range_fits(rns8_semantics s, const I512& bound, const I256& product) {
  if (bound.negative()) return false;
  const I512 p = I512::widen(product);
  return s == RNS8_EXACT_WIDE_SIGNED ? (bound + bound) < p : bound < p;
}

// exact_range.hpp:34-47
inline void add_exact_value(ExactAxis& a, const I512& v, bool first) {
  const I512 mag = v.abs();
  a.max_magnitude = imax(a.max_magnitude, mag);
  a.absolute_sum = a.absolute_sum + mag;
  a.sum = a.sum + v;
  if (first) {
    a.minimum = v;
    a.maximum = v;
  } else {
    a.minimum = imin(a.minimum, v);
    a.maximum = imax(a.maximum, v);
  }
  a.sum_known = true;
}

// exact_range.hpp:24-32
inline I512 axis_center(const ExactAxis& a) { return (a.minimum + a.maximum).half_trunc(); }
inline I512 axis_deviation_max(const ExactAxis& a, const I512& c) {
  return imax((a.minimum - c).abs(), (a.maximum - c).abs());
}

// exact_range.hpp:52-78: summaries of a host operand, two linear scans.
// Every quantity of a 64-bit operand fits 128 bits (sums of fewer than 2^63
// magnitudes below 2^64), so the scans accumulate in __int128 over row
// shards on up to `max_threads` threads, merge the column partials, and
// widen to I512 at the end: the same integers as summing in I512.
namespace native_detail {
struct Acc {
  unsigned __int128 max_magnitude = 0, absolute_sum = 0, deviation_sum = 0;
  __int128 sum = 0, minimum = 0, maximum = 0;
  bool any = false;
  void add(__int128 v) {
    const unsigned __int128 mag = static_cast<unsigned __int128>(v < 0 ? -v : v);
    max_magnitude = mag > max_magnitude ? mag : max_magnitude;
    absolute_sum += mag;
    sum += v;
    minimum = !any || v < minimum ? v : minimum;
    maximum = !any || v > maximum ? v : maximum;
    any = true;
  }
  void merge(const Acc& o) {
    if (!o.any) return;
    max_magnitude = o.max_magnitude > max_magnitude ? o.max_magnitude : max_magnitude;
    absolute_sum += o.absolute_sum;
    deviation_sum += o.deviation_sum;
    sum += o.sum;
    minimum = !any || o.minimum < minimum ? o.minimum : minimum;
    maximum = !any || o.maximum > maximum ? o.maximum : maximum;
    any = true;
  }
  // (min + max) / 2 truncated toward zero, as C++ integer division does
  __int128 center() const { return (minimum + maximum) / 2; }
};
inline I512 from_u128(unsigned __int128 v) {
  I512 r;
  r.w[0] = static_cast<uint64_t>(v);
  r.w[1] = static_cast<uint64_t>(v >> 64);
  return r;
}
inline I512 from_i128(__int128 v) {
  const I512 m = from_u128(static_cast<unsigned __int128>(v < 0 ? -v : v));
  return v < 0 ? -m : m;
}
inline ExactAxis widen_axis(const Acc& a) {
  ExactAxis e;
  e.max_magnitude = from_u128(a.max_magnitude);
  e.absolute_sum = from_u128(a.absolute_sum);
  e.sum = from_i128(a.sum);
  e.minimum = from_i128(a.minimum);
  e.maximum = from_i128(a.maximum);
  e.deviation_sum = from_u128(a.deviation_sum);
  e.sum_known = a.any;
  return e;
}
}  // namespace native_detail

template <typename T>
void native_exact_ranges(const T* src, int64_t rows, int64_t cols, int64_t ld, I512& maximum,
                         std::vector<ExactAxis>& row_axes, std::vector<ExactAxis>& col_axes,
                         unsigned max_threads = 16) {
  using native_detail::Acc;
  auto value = [&](int64_t r, int64_t c) -> __int128 {
    return std::is_signed<T>::value ? static_cast<__int128>(static_cast<int64_t>(src[r * ld + c]))
                                    : static_cast<__int128>(static_cast<uint64_t>(src[r * ld + c]));
  };
  unsigned nt = std::max(1u, std::min(max_threads, std::thread::hardware_concurrency()));
  if (static_cast<int64_t>(nt) > rows) nt = static_cast<unsigned>(std::max<int64_t>(rows, 1));
  std::vector<Acc> racc(static_cast<std::size_t>(rows)), cacc(static_cast<std::size_t>(cols));
  std::vector<std::vector<Acc>> cpart(nt, std::vector<Acc>(static_cast<std::size_t>(cols)));
  // pass 1: row accumulators, and column partials per shard
  run_shards(nt, [&](unsigned t) {
    const int64_t r0 = rows * t / nt, r1 = rows * (t + 1) / nt;
    for (int64_t r = r0; r < r1; ++r)
      for (int64_t c = 0; c < cols; ++c) {
        const __int128 v = value(r, c);
        racc[r].add(v);
        cpart[t][c].add(v);
      }
  });
  for (unsigned t = 0; t < nt; ++t)
    for (int64_t c = 0; c < cols; ++c) cacc[c].merge(cpart[t][c]);
  // pass 2: deviation sums around the row and column centres
  std::vector<__int128> ccenter(static_cast<std::size_t>(cols));
  for (int64_t c = 0; c < cols; ++c) ccenter[c] = cacc[c].center();
  std::vector<std::vector<unsigned __int128>> cdev(nt, std::vector<unsigned __int128>(static_cast<std::size_t>(cols)));
  run_shards(nt, [&](unsigned t) {
    const int64_t r0 = rows * t / nt, r1 = rows * (t + 1) / nt;
    for (int64_t r = r0; r < r1; ++r) {
      const __int128 rc = racc[r].center();
      unsigned __int128 dev = 0;
      for (int64_t c = 0; c < cols; ++c) {
        const __int128 v = value(r, c);
        const __int128 dr = v - rc, dc = v - ccenter[c];
        dev += static_cast<unsigned __int128>(dr < 0 ? -dr : dr);
        cdev[t][c] += static_cast<unsigned __int128>(dc < 0 ? -dc : dc);
      }
      racc[r].deviation_sum = dev;
    }
  });
  for (unsigned t = 0; t < nt; ++t)
    for (int64_t c = 0; c < cols; ++c) cacc[c].deviation_sum += cdev[t][c];
  row_axes.resize(static_cast<std::size_t>(rows));
  col_axes.resize(static_cast<std::size_t>(cols));
  unsigned __int128 top = 0;
  for (int64_t r = 0; r < rows; ++r) {
    row_axes[r] = native_detail::widen_axis(racc[r]);
    top = racc[r].max_magnitude > top ? racc[r].max_magnitude : top;
  }
  for (int64_t c = 0; c < cols; ++c) col_axes[c] = native_detail::widen_axis(cacc[c]);
  maximum = native_detail::from_u128(top);
}

// exact_range.hpp:80-99: a bound on |dot(row, column)| of length k.
inline I512 axis_product_bound(const ExactAxis& a, const ExactAxis& b, int64_t k) {
  const I512 kk = I512::from_u64(static_cast<uint64_t>(k));
  I512 bound = kk * a.max_magnitude * b.max_magnitude;
  bound = imin(bound, a.absolute_sum * b.max_magnitude);
  bound = imin(bound, a.max_magnitude * b.absolute_sum);
  if (a.sum_known && b.sum_known) {
    const I512 ca = axis_center(a), cb = axis_center(b);
    const I512 da = axis_deviation_max(a, ca), db = axis_deviation_max(b, cb);
    I512 rem = kk * da * db;
    rem = imin(rem, a.deviation_sum * db);
    rem = imin(rem, da * b.deviation_sum);
    const I512 center_term = ca * b.sum + cb * a.sum - kk * ca * cb;
    bound = imin(bound, center_term.abs() + rem);
  }
  return bound;
}

// exact_range.hpp:101-106
inline ExactAxis uniform_axis(const I512& maximum, int64_t length) {
  ExactAxis a;
  a.max_magnitude = maximum;
  a.absolute_sum = I512::from_u64(static_cast<uint64_t>(length)) * maximum;
  return a;
}

// axis_product_bound with the factors that depend on one axis only computed
// once per row or column (the centre, the deviation maximum and their
// products with k): the same integers, so the same bound.
struct AxisTerms {
  I512 max_magnitude, absolute_sum, k_max;
  bool sum_known = false;
  I512 sum, center, deviation, deviation_sum, k_center, k_deviation;
};
inline AxisTerms axis_terms(const ExactAxis& a, int64_t k) {
  const I512 kk = I512::from_u64(static_cast<uint64_t>(k));
  AxisTerms t;
  t.max_magnitude = a.max_magnitude;
  t.absolute_sum = a.absolute_sum;
  t.k_max = kk * a.max_magnitude;
  t.sum_known = a.sum_known;
  if (a.sum_known) {
    t.sum = a.sum;
    t.center = axis_center(a);
    t.deviation = axis_deviation_max(a, t.center);
    t.deviation_sum = a.deviation_sum;
    t.k_center = kk * t.center;
    t.k_deviation = kk * t.deviation;
  }
  return t;
}
inline I512 cell_bound(const AxisTerms& a, const AxisTerms& b) {
  I512 bound = a.k_max * b.max_magnitude;
  bound = imin(bound, a.absolute_sum * b.max_magnitude);
  bound = imin(bound, a.max_magnitude * b.absolute_sum);
  if (a.sum_known && b.sum_known) {
    I512 rem = a.k_deviation * b.deviation;
    rem = imin(rem, a.deviation_sum * b.deviation);
    rem = imin(rem, a.deviation * b.deviation_sum);
    const I512 center_term = a.center * b.sum + b.center * a.sum - a.k_center * b.center;
    bound = imin(bound, center_term.abs() + rem);
  }
  return bound;
}

// What a packed exact-wide operand carries into a GEMM.
struct ExactOperand {
  const I512* max_magnitude;
  const std::vector<ExactAxis>* rows;  // per-row summaries (may be empty)
  const std::vector<ExactAxis>* cols;  // per-column summaries (may be empty)
};

// exact_range.hpp:104-157: output bound of C = A x B (m x n, inner k), the
// per-row / per-column summaries C carries into a later GEMM, and the
// admission decision against the modulus product. Rows are independent and
// are split over up to `max_threads` host threads.
inline rns8_status exact_product_range(rns8_semantics semantics, int64_t m, int64_t n, int64_t k,
                                       const ExactOperand& A, const ExactOperand& B, const I256& product,
                                       I512& bound, std::vector<ExactAxis>* out_rows,
                                       std::vector<ExactAxis>* out_cols, unsigned max_threads = 16) {
  const bool a_rows = A.rows->size() == static_cast<std::size_t>(m);
  const bool b_cols = B.cols->size() == static_cast<std::size_t>(n);
  bound = I512::from_u64(static_cast<uint64_t>(k)) * *A.max_magnitude * *B.max_magnitude;
  if (out_rows) out_rows->clear();
  if (out_cols) out_cols->clear();
  if (a_rows || b_cols) {
    const AxisTerms fa = axis_terms(uniform_axis(*A.max_magnitude, k), k);
    const AxisTerms fb = axis_terms(uniform_axis(*B.max_magnitude, k), k);
    std::vector<AxisTerms> ta(a_rows ? static_cast<std::size_t>(m) : 0u), tb(b_cols ? static_cast<std::size_t>(n) : 0u);
    for (std::size_t r = 0; r < ta.size(); ++r) ta[r] = axis_terms((*A.rows)[r], k);
    for (std::size_t c = 0; c < tb.size(); ++c) tb[c] = axis_terms((*B.cols)[c], k);
    std::vector<ExactAxis> rows(static_cast<std::size_t>(m)), cols(static_cast<std::size_t>(n));
    // column summaries are merged per thread, then reduced
    unsigned nt = std::max(1u, std::min(max_threads, std::thread::hardware_concurrency()));
    if (static_cast<int64_t>(nt) > m) nt = static_cast<unsigned>(m);
    std::vector<std::vector<ExactAxis>> col_parts(nt, std::vector<ExactAxis>(static_cast<std::size_t>(n)));
    std::vector<I512> maxima(nt);
    auto work = [&](unsigned t) {
      const int64_t r0 = m * t / nt, r1 = m * (t + 1) / nt;
      for (int64_t r = r0; r < r1; ++r) {
        const AxisTerms& a = a_rows ? ta[r] : fa;
        for (int64_t c = 0; c < n; ++c) {
          const AxisTerms& b = b_cols ? tb[c] : fb;
          const I512 cell = cell_bound(a, b);
          maxima[t] = imax(maxima[t], cell);
          rows[r].max_magnitude = imax(rows[r].max_magnitude, cell);
          rows[r].absolute_sum = rows[r].absolute_sum + cell;
          ExactAxis& cc = col_parts[t][c];
          cc.max_magnitude = imax(cc.max_magnitude, cell);
          cc.absolute_sum = cc.absolute_sum + cell;
        }
      }
    };
    run_shards(nt, work);
    I512 maximum;
    for (unsigned t = 0; t < nt; ++t) {
      maximum = imax(maximum, maxima[t]);
      for (int64_t c = 0; c < n; ++c) {
        cols[c].max_magnitude = imax(cols[c].max_magnitude, col_parts[t][c].max_magnitude);
        cols[c].absolute_sum = cols[c].absolute_sum + col_parts[t][c].absolute_sum;
      }
    }
    bound = imin(bound, maximum);
    if (out_rows) out_rows->swap(rows);
    if (out_cols) out_cols->swap(cols);
  }
  return exact_range_fits(semantics, bound, product) ? RNS8_SUCCESS : RNS8_RANGE_ERROR;
}

}  // namespace rns8x
