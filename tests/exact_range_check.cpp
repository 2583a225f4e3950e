// Host check of the library's exact-wide proof arithmetic
// (rns8_amd/csrc/exact_axes.hpp, the header exact_axes.hip's kernels are
// built from): reads cases from stdin and prints what the device computes,
// for tests/test_exact_range_host.py to compare with the Python-integer
// restatement in oracle/exact_range.py.
//
// Numbers are signed hexadecimal ("-1f"). Three kinds of case:
//
//   case <S|U> <m> <n> <k> <product>
//   <A max> <rows r> then r axes, <B max> <cols c> then c axes
//     an axis: max_magnitude absolute_sum sum minimum maximum deviation_sum
//     sum_known(0/1). A's rows are native axes when sum_known is set,
//     carried otherwise, and uniform when r != m (likewise B's columns).
//     Output: "<status> <bound>", then (unless both sides are uniform) m
//     lines "<row max> <row absolute sum>" and n lines for the columns.
//     Quantities at or above 2^256 print as 2^256 - 1 (the kernels saturate).
//
//   ops <a> <b>
//     for 0 <= a, b < 2^256: sat_mul, sat_add, min and max.
//
//   native <S|U> <rows> <cols> then rows x cols values
//     the summaries of a 64-bit operand, computed in the device passes'
//     decomposition (per 64 x 64 tile partials of each row and column,
//     extremes as maxima of biased values, merged per axis) with the same
//     functions. Output: max |x|, then one line per row and per column with
//     the seven fields above.
#include <cstdint>
#include <cstdio>
#include <iostream>
#include <string>
#include <vector>

#include "exact_axes.hpp"
#include "exact_range.hpp"

using namespace rns8x;
using namespace rns8x::xa;

namespace {

// |value| < 2^256 with its sign
struct Parsed {
  bool neg = false;
  U256 mag = zero256();
};

Parsed parse(const std::string& s) {
  Parsed p;
  p.neg = !s.empty() && s[0] == '-';
  for (std::size_t i = p.neg ? 1 : 0; i < s.size(); ++i) {
    const char ch = s[i];
    const u64 d = ch <= '9' ? ch - '0' : (ch | 0x20) - 'a' + 10;
    if (p.mag.w[3] >> 60) {
      std::fprintf(stderr, "value above 2^256\n");
      std::exit(3);
    }
    for (int w = 3; w > 0; --w) p.mag.w[w] = (p.mag.w[w] << 4) | (p.mag.w[w - 1] >> 60);
    p.mag.w[0] = (p.mag.w[0] << 4) | d;
  }
  return p;
}

i128 to_i128(const Parsed& p) {
  const i128 m = static_cast<i128>(get_u128(p.mag.w));
  return p.neg ? -m : m;
}

std::string hex(const U256& v) {
  std::string out;
  bool started = false;
  for (int i = 3; i >= 0; --i) {
    char buf[20];
    if (!started) {
      if (!v.w[i] && i) continue;
      std::snprintf(buf, sizeof buf, "%llx", static_cast<unsigned long long>(v.w[i]));
      started = true;
    } else {
      std::snprintf(buf, sizeof buf, "%016llx", static_cast<unsigned long long>(v.w[i]));
    }
    out += buf;
  }
  return out;
}
std::string hex_i128(i128 v) {
  const u128 m = static_cast<u128>(v < 0 ? -v : v);
  return (v < 0 ? "-" : "") + hex(from128(m));
}

AxisRecord read_axis(bool& sum_known) {
  std::string f[7];
  for (auto& x : f) std::cin >> x;
  AxisRecord r{};
  put_u256(r.max_magnitude, parse(f[0]).mag);
  put_u256(r.absolute_sum, parse(f[1]).mag);
  sum_known = f[6] == "1";
  if (sum_known) {
    put_u128(r.sum, static_cast<u128>(to_i128(parse(f[2]))));
    put_u128(r.minimum, static_cast<u128>(to_i128(parse(f[3]))));
    put_u128(r.maximum, static_cast<u128>(to_i128(parse(f[4]))));
    put_u128(r.deviation_sum, get_u128(parse(f[5]).mag.w));
  }
  return r;
}

I512 widen(const U256& v) {
  I512 r;
  for (int i = 0; i < 4; ++i) r.w[i] = v.w[i];
  return r;
}

int gemm_case() {
  std::string sem, ps, as, bs;
  int64_t m, n, k;
  std::size_t count;
  std::cin >> sem >> m >> n >> k >> ps;
  I256 product;
  {
    const U256 p = parse(ps).mag;
    for (int i = 0; i < 4; ++i) product.w[i] = p.w[i];
  }
  auto side = [&](std::string& mx, int64_t want, std::vector<AxisRecord>& recs, AxisKind& kind) {
    std::cin >> mx >> count;
    recs.resize(count);
    bool known = false;
    for (auto& r : recs) r = read_axis(known);
    kind = static_cast<int64_t>(count) != want ? AxisKind::Uniform : known ? AxisKind::Native : AxisKind::Carried;
  };
  std::vector<AxisRecord> arows, bcols;
  AxisKind ak, bk;
  side(as, m, arows, ak);
  side(bs, n, bcols, bk);
  const U256 amax = parse(as).mag, bmax = parse(bs).mag;
  std::vector<U256> rmax(m, zero256()), rsum(m, zero256()), cmax(n, zero256()), csum(n, zero256());
  U256 top = zero256();
  for (int64_t r = 0; r < m; ++r) {
    const AxisTerms a = axis_terms(ak == AxisKind::Uniform ? nullptr : &arows[r], ak, amax, static_cast<u64>(k));
    for (int64_t c = 0; c < n; ++c) {
      const AxisTerms b = axis_terms(bk == AxisKind::Uniform ? nullptr : &bcols[c], bk, bmax, static_cast<u64>(k));
      const U256 cell = cell_bound(a, b);
      rmax[r] = max256(rmax[r], cell);
      rsum[r] = sat_add(rsum[r], cell);
      cmax[c] = max256(cmax[c], cell);
      csum[c] = sat_add(csum[c], cell);
      top = max256(top, cell);
    }
  }
  const U256 bound = min256(sat_mul(sat_mul64(static_cast<u64>(k), amax), bmax), top);
  const rns8_semantics s = sem == "S" ? RNS8_EXACT_WIDE_SIGNED : RNS8_EXACT_WIDE_UNSIGNED;
  const int st = exact_range_fits(s, widen(bound), product) ? 0 : 5;
  std::cout << st << " " << hex(bound) << "\n";
  if (ak == AxisKind::Uniform && bk == AxisKind::Uniform) return 0;
  for (int64_t r = 0; r < m; ++r) std::cout << hex(rmax[r]) << " " << hex(rsum[r]) << "\n";
  for (int64_t c = 0; c < n; ++c) std::cout << hex(cmax[c]) << " " << hex(csum[c]) << "\n";
  return 0;
}

// The device passes' decomposition (exact_axes.hip native_axes_pass and
// native_axes_finish): per 64 x 64 tile, each row's and each column's
// partial over two halves of 32, merged; then each axis's partials merged in
// tile order, the record built, and a second pass of deviation partials
// around the records' centres.
int native_case() {
  std::string sem;
  int64_t rows, cols;
  std::cin >> sem >> rows >> cols;
  const bool sgn = sem == "S";
  std::vector<u64> xs(static_cast<std::size_t>(rows * cols));
  for (auto& x : xs) {
    std::string v;
    std::cin >> v;
    const Parsed p = parse(v);
    x = p.neg ? u64{0} - p.mag.w[0] : p.mag.w[0];
  }
  const int T = 64;
  const int64_t tx = (cols + T - 1) / T, ty = (rows + T - 1) / T;
  std::vector<AxisPartial> rpart(rows * tx), cpart(cols * ty);
  std::vector<AxisRecord> rr(rows), cr(cols);
  for (int pass = 0; pass < 2; ++pass) {
    for (int64_t y = 0; y < ty; ++y)
      for (int64_t x = 0; x < tx; ++x) {
        const int64_t r0 = y * T, c0 = x * T;
        const int64_t nr = rows - r0 < T ? rows - r0 : T, nc = cols - c0 < T ? cols - c0 : T;
        for (int by_row = 1; by_row >= 0; --by_row)
          for (int64_t lane = 0; lane < (by_row ? nr : nc); ++lane) {
            const int64_t len = by_row ? nc : nr;
            auto at = [&](int64_t j) {
              return by_row ? xs[(r0 + lane) * cols + c0 + j] : xs[(r0 + j) * cols + c0 + lane];
            };
            AxisPartial halves[2] = {empty_partial(), empty_partial()};
            for (int h = 0; h < 2; ++h) {
              PartialAcc acc;
              DeviationAcc dev;
              for (int64_t j = 32 * h; j < len && j < 32 * h + 32; ++j) {
                if (pass == 0)
                  acc.add(at(j), sgn);
                else
                  dev.add(deviation(at(j), record_centre(by_row ? rr[r0 + lane] : cr[c0 + lane]), sgn));
              }
              if (pass == 0) halves[h] = acc.partial();
              else halves[h].sum = dev.value();
            }
            partial_merge(halves[0], halves[1]);
            (by_row ? rpart[x * rows + r0 + lane] : cpart[y * cols + c0 + lane]) = halves[0];
          }
      }
    for (int by_row = 1; by_row >= 0; --by_row)
      for (int64_t axis = 0; axis < (by_row ? rows : cols); ++axis) {
        const int64_t parts = by_row ? tx : ty, stride = by_row ? rows : cols;
        const AxisPartial* part = by_row ? &rpart[axis] : &cpart[axis];
        AxisRecord& rec = by_row ? rr[axis] : cr[axis];
        if (pass == 0) {
          AxisPartial p = part[0];
          for (int64_t t = 1; t < parts; ++t) partial_merge(p, part[t * stride]);
          rec = native_record(p, static_cast<u64>(by_row ? cols : rows), sgn);
        } else {
          u128 dev = 0;
          for (int64_t t = 0; t < parts; ++t) dev += part[t * stride].sum;
          put_u128(rec.deviation_sum, dev);
        }
      }
  }
  u64 top = 0;
  for (const auto& r : rr) top = r.max_magnitude[0] > top ? r.max_magnitude[0] : top;
  std::cout << hex(from128(top)) << "\n";
  auto print = [](const AxisRecord& a) {
    std::cout << hex(get_u256(a.max_magnitude)) << " " << hex(get_u256(a.absolute_sum)) << " "
              << hex_i128(get_i128(a.sum)) << " " << hex_i128(get_i128(a.minimum)) << " "
              << hex_i128(get_i128(a.maximum)) << " " << hex(from128(get_u128(a.deviation_sum))) << " 1\n";
  };
  for (const auto& a : rr) print(a);
  for (const auto& a : cr) print(a);
  return 0;
}

// ops <a> <b> (both below 2^256): sat_mul, sat_add, min and max on one line
int ops_case() {
  std::string as, bs;
  std::cin >> as >> bs;
  const U256 a = parse(as).mag, b = parse(bs).mag;
  std::cout << hex(sat_mul(a, b)) << " " << hex(sat_add(a, b)) << " " << hex(min256(a, b)) << " "
            << hex(max256(a, b)) << "\n";
  return 0;
}

}  // namespace

int main() {
  std::string tag;
  while (std::cin >> tag) {
    if (tag == "native") native_case();
    else if (tag == "case") gemm_case();
    else if (tag == "ops") ops_case();
    else return 2;
  }
  return 0;
}
