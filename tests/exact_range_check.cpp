// Host check of the library's exact-wide admission math
// (rns8_amd/csrc/exact_range.hpp, the header librns8.so is built from): reads
// GEMM cases from stdin and prints the bound, the admission status and the
// summaries the product carries, for tests/test_exact_range_host.py to compare
// with the Python-integer restatement in oracle/exact_range.py.
//
// Input, whitespace separated, numbers in signed hexadecimal ("-1f"):
//   case <S|U> <m> <n> <k> <product>
//   <A max> <rows r> then r axes, <B max> <cols c> then c axes
// where an axis is: max_magnitude absolute_sum sum minimum maximum
// deviation_sum sum_known(0/1). Output per case:
//   <status> <bound>
//   m lines "<row max> <row absolute sum>", n lines for the columns
// (no summaries are printed when the product carries none).
#include <cstdint>
#include <cstdio>
#include <iostream>
#include <string>
#include <vector>

#include "exact_range.hpp"

using rns8x::I256;
using rns8x::I512;

namespace {

template <typename W>
W parse(const std::string& s) {
  const bool neg = !s.empty() && s[0] == '-';
  W v;
  for (std::size_t i = neg ? 1 : 0; i < s.size(); ++i) {
    const char ch = s[i];
    const uint64_t d = ch <= '9' ? ch - '0' : (ch | 0x20) - 'a' + 10;
    v = v * W::from_u64(16) + W::from_u64(d);
  }
  return neg ? -v : v;
}

std::string hex(const I512& v) {
  if (v.negative()) return "-" + hex(-v);
  std::string out;
  bool started = false;
  for (int i = static_cast<int>(sizeof(v.w) / sizeof(v.w[0])) - 1; i >= 0; --i) {
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

ExactAxis read_axis() {
  std::string f[7];
  for (auto& x : f) std::cin >> x;
  ExactAxis a;
  a.max_magnitude = parse<I512>(f[0]);
  a.absolute_sum = parse<I512>(f[1]);
  a.sum = parse<I512>(f[2]);
  a.minimum = parse<I512>(f[3]);
  a.maximum = parse<I512>(f[4]);
  a.deviation_sum = parse<I512>(f[5]);
  a.sum_known = f[6] == "1";
  return a;
}

void print_axis(const ExactAxis& a) {
  std::cout << hex(a.max_magnitude) << " " << hex(a.absolute_sum) << " " << hex(a.sum) << " " << hex(a.minimum) << " "
            << hex(a.maximum) << " " << hex(a.deviation_sum) << " " << (a.sum_known ? 1 : 0) << "\n";
}

// native <S|U> <rows> <cols> then rows x cols values: the summaries of a host
// operand (native_exact_ranges), max then one line per row and per column
int native_case() {
  std::string sem;
  int64_t rows, cols;
  std::cin >> sem >> rows >> cols;
  std::vector<int64_t> xs(static_cast<std::size_t>(rows * cols));
  for (auto& x : xs) {
    std::string v;
    std::cin >> v;
    x = static_cast<int64_t>(parse<I512>(v).w[0]);
  }
  I512 maximum;
  std::vector<ExactAxis> ra, ca;
  if (sem == "S")
    rns8x::native_exact_ranges(xs.data(), rows, cols, cols, maximum, ra, ca, 3);
  else
    rns8x::native_exact_ranges(reinterpret_cast<const uint64_t*>(xs.data()), rows, cols, cols, maximum, ra, ca, 3);
  std::cout << hex(maximum) << "\n";
  for (const auto& a : ra) print_axis(a);
  for (const auto& a : ca) print_axis(a);
  return 0;
}

}  // namespace

int main() {
  std::string tag;
  while (std::cin >> tag) {
    if (tag == "native") {
      native_case();
      continue;
    }
    if (tag != "case") return 2;
    std::string sem, ps, as, bs;
    int64_t m, n, k;
    std::cin >> sem >> m >> n >> k >> ps;
    const I256 product = parse<I256>(ps);
    std::size_t count;
    std::cin >> as >> count;
    const I512 amax = parse<I512>(as);
    std::vector<ExactAxis> arows(count), none;
    for (auto& a : arows) a = read_axis();
    std::cin >> bs >> count;
    const I512 bmax = parse<I512>(bs);
    std::vector<ExactAxis> bcols(count);
    for (auto& b : bcols) b = read_axis();
    const rns8x::ExactOperand A{&amax, &arows, &none};
    const rns8x::ExactOperand B{&bmax, &none, &bcols};
    I512 bound;
    std::vector<ExactAxis> rows, cols;
    const rns8_semantics s = sem == "S" ? RNS8_EXACT_WIDE_SIGNED : RNS8_EXACT_WIDE_UNSIGNED;
    const rns8_status st = rns8x::exact_product_range(s, m, n, k, A, B, product, bound, &rows, &cols, 4);
    std::cout << static_cast<int>(st) << " " << hex(bound) << "\n";
    for (const auto& r : rows) std::cout << hex(r.max_magnitude) << " " << hex(r.absolute_sum) << "\n";
    for (const auto& c : cols) std::cout << hex(c.max_magnitude) << " " << hex(c.absolute_sum) << "\n";
  }
  return 0;
}
