// The exact-wide admission rule (reference src/core/exact_range.hpp:16-18):
// a bound on |C| is admitted at a prefix iff 2 * bound < P for signed
// results and bound < P for unsigned ones, P the prefix's modulus product.
// The bounds themselves (per-axis summaries and cell bounds) are computed on
// the device: exact_axes.hpp / exact_axes.hip, driven by exact_proof.cpp.
#pragma once

#include "rns8/rns8.h"
#include "wide_int.hpp"

namespace rns8x {

inline bool exact_range_fits(rns8_semantics s, const I512& bound, const I256& product) {
  if (bound.negative()) return false;
  const I512 p = I512::widen(product);
  return s == RNS8_EXACT_WIDE_SIGNED ? (bound + bound) < p : bound < p;
}

}  // namespace rns8x
