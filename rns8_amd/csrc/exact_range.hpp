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
template <typename T>
void native_exact_ranges(const T* src, int64_t rows, int64_t cols, int64_t ld, I512& maximum,
                         std::vector<ExactAxis>& row_axes, std::vector<ExactAxis>& col_axes) {
  row_axes.assign(static_cast<std::size_t>(rows), ExactAxis{});
  col_axes.assign(static_cast<std::size_t>(cols), ExactAxis{});
  auto value = [](T x) {
    return std::is_signed<T>::value ? I512::from_i64(static_cast<int64_t>(x))
                                    : I512::from_u64(static_cast<uint64_t>(x));
  };
  maximum = I512();
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      const I512 v = value(src[r * ld + c]);
      add_exact_value(row_axes[r], v, c == 0);
      add_exact_value(col_axes[c], v, r == 0);
    }
    maximum = imax(maximum, row_axes[r].max_magnitude);
  }
  std::vector<I512> col_center(static_cast<std::size_t>(cols));
  for (int64_t c = 0; c < cols; ++c) col_center[c] = axis_center(col_axes[c]);
  for (int64_t r = 0; r < rows; ++r) {
    const I512 rc = axis_center(row_axes[r]);
    for (int64_t c = 0; c < cols; ++c) {
      const I512 v = value(src[r * ld + c]);
      row_axes[r].deviation_sum = row_axes[r].deviation_sum + (v - rc).abs();
      col_axes[c].deviation_sum = col_axes[c].deviation_sum + (v - col_center[c]).abs();
    }
  }
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
    const ExactAxis fa = uniform_axis(*A.max_magnitude, k);
    const ExactAxis fb = uniform_axis(*B.max_magnitude, k);
    std::vector<ExactAxis> rows(static_cast<std::size_t>(m)), cols(static_cast<std::size_t>(n));
    // column summaries are merged per thread, then reduced
    unsigned nt = std::max(1u, std::min(max_threads, std::thread::hardware_concurrency()));
    if (static_cast<int64_t>(nt) > m) nt = static_cast<unsigned>(m);
    std::vector<std::vector<ExactAxis>> col_parts(nt, std::vector<ExactAxis>(static_cast<std::size_t>(n)));
    std::vector<I512> maxima(nt);
    auto work = [&](unsigned t) {
      const int64_t r0 = m * t / nt, r1 = m * (t + 1) / nt;
      for (int64_t r = r0; r < r1; ++r) {
        const ExactAxis& a = a_rows ? (*A.rows)[r] : fa;
        for (int64_t c = 0; c < n; ++c) {
          const ExactAxis& b = b_cols ? (*B.cols)[c] : fb;
          const I512 cell = axis_product_bound(a, b, k);
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
