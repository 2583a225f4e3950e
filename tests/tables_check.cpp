// Host check of the constant tables in rns8_amd/csrc/tables.hpp and of the
// integer steps the gfx950 kernels run on them, emulated instruction by
// instruction:
//   udot4(a, b, c)   = c + sum_k byte_k(a) * byte_k(b)  (mod 2^32)  v_dot4_u32_u8
//   umulhi(x, y)     = (x * y) >> 32                               v_mul_hi_u32
//   mulhi_u24(x, y)  = (lo24(x) * lo24(y)) >> 32                   v_mul_hi_u32_u24
//   mad_u24(a, b, c) = lo24(a) * lo24(b) + c  (mod 2^32)           v_mad_u32_u24
//   perm(s0, s1, sel): result byte k = byte sel_k of s1 (0-3), of s0 (4-7),
//                      0 for selector 0x0c                         v_perm_b32
// Expected values are computed independently with 64/128-bit '%'. Modes:
//   quot      exhaustive quotient checks for every modulus 2..256
//   reduce32  int32 accumulator -> packed centered int8 (GEMM epilogue)
//   pack64    int64 / uint64 -> centered residue (pack kernel)
//   garner    prints Garner tables and digit vectors for a big-int check
//   div       unit-index division: make_div_u31 over n < 2^31
//   export64  the int64 / uint64 export tail at every prefix around the
//             64-bit edges, against __int128 arithmetic
//   crt       prints the CRT-basis export tables (crt_export.hpp) of every
//             prefix, then reads residue vectors ("P r_0 .. r_{P-1}" lines)
//             from stdin and prints the centered value the export tail
//             computes from their column sums; tests/test_tables.py checks
//             both against Python big integers
//   crtgate   the address limits of the CRT-basis export kernel
//   crt64     the 64-bit CRT tail at P = 9..11 against __int128 values
// Exit status 0 and a final "ok" line when every check passes.
#include <cinttypes>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <utility>
#include <vector>

#include "crt_export.hpp"
#include "tables.hpp"

using namespace rns8x;

namespace {

uint32_t udot4(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t s = c;
  for (int k = 0; k < 4; ++k) s += ((a >> (8 * k)) & 0xFFu) * ((b >> (8 * k)) & 0xFFu);
  return s;
}
uint32_t umulhi(uint32_t x, uint32_t y) { return static_cast<uint32_t>((uint64_t{x} * y) >> 32); }
uint32_t mulhi_u24(uint32_t x, uint32_t y) {
  return static_cast<uint32_t>((uint64_t{x & 0xFFFFFFu} * (y & 0xFFFFFFu)) >> 32);
}
uint32_t mad_u24(uint32_t a, uint32_t b, uint32_t c) { return (a & 0xFFFFFFu) * (b & 0xFFFFFFu) + c; }
uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  const uint64_t both = (uint64_t{s0} << 32) | s1;
  uint32_t out = 0;
  for (int k = 0; k < 4; ++k) {
    const uint32_t sk = (sel >> (8 * k)) & 0xFFu;
    uint32_t byte = 0;
    if (sk < 8) byte = static_cast<uint32_t>((both >> (8 * sk)) & 0xFFu);
    else if (sk == 0x0c) byte = 0;
    else std::abort();  // selectors the kernels do not use
    out |= byte << (8 * k);
  }
  return out;
}

// SplitMix64 for reproducible random cases.
struct Rng {
  uint64_t s;
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
};

int64_t centered_ref(__int128 x, uint32_t m) {
  const __int128 h = m / 2;
  __int128 r = (x + h) % m;
  if (r < 0) r += m;
  return static_cast<int64_t>(r - h);
}

int failures = 0;
void fail(const char* what, uint32_t m, long long a, long long b, long long c) {
  if (failures < 20) std::printf("FAIL %s m=%u %lld %lld %lld\n", what, m, a, b, c);
  ++failures;
}

uint32_t s_max_i32(const ModulusConsts& c) {
  uint32_t bytes = 0;
  for (int k = 0; k < 4; ++k) bytes += (c.pow_lo >> (8 * k)) & 0xFFu;
  return 255u * bytes + c.off_i32;
}

void check_quot() {
  uint64_t checks = 0;
  for (uint32_t m = 2; m <= 256; ++m) {
    const ModulusConsts c = make_modulus_consts(m);
    const uint32_t smax = s_max_i32(c);
    if (smax >= (1u << 20)) fail("smax", m, smax, 0, 0);
    if ((uint64_t{smax} << c.q_shift) >= (1u << 24)) fail("shifted smax", m, smax, c.q_shift, 0);
    if (c.q_recip >= (1u << 24)) fail("recip24", m, c.q_recip, 0, 0);
    for (uint32_t s = 0; s <= smax; ++s, ++checks)
      if (mulhi_u24(s << c.q_shift, c.q_recip) != s / m) fail("quot24", m, s, mulhi_u24(s << c.q_shift, c.q_recip), s / m);
    // byte weights, computed independently
    for (uint32_t b = 0; b < 4; ++b) {
      const uint64_t lo = (uint64_t{1} << (8 * b)) % m;
      const uint64_t hi = static_cast<uint64_t>((static_cast<unsigned __int128>(1) << (32 + 8 * b)) % m);
      if (((c.pow_lo >> (8 * b)) & 0xFFu) != lo) fail("pow_lo", m, b, c.pow_lo, lo);
      if (((c.pow_hi >> (8 * b)) & 0xFFu) != hi) fail("pow_hi", m, b, c.pow_hi, hi);
    }
    // pack reduction of a 64-bit value: two byte dot products plus an offset
    uint32_t hbytes = 0;
    for (int k = 0; k < 4; ++k) hbytes += ((c.pow_lo >> (8 * k)) & 0xFFu) + ((c.pow_hi >> (8 * k)) & 0xFFu);
    const uint32_t pmax = 255u * hbytes + (c.off_i64 > c.off_u64 ? c.off_i64 : c.off_u64);
    if ((uint64_t{pmax} << c.pq_shift) >= (1u << 24) || c.pq_recip >= (1u << 24)) fail("pack quot range", m, pmax, 0, 0);
    for (uint32_t s = 0; s <= pmax; ++s, ++checks)
      if (mulhi_u24(s << c.pq_shift, c.pq_recip) != s / m) fail("pack quot24", m, s, 0, 0);
    // 32-bit reciprocal kept for host use: exact below 2^21
    for (uint32_t s = 0; s < (1u << 21); ++s, ++checks)
      if (umulhi(s, c.recip) != s / m) fail("quot32", m, s, umulhi(s, c.recip), s / m);
  }
  std::printf("quot checks %" PRIu64 "\n", checks);
}

// centered_byte (int_ops.hpp): sc = s - H with s congruent to x + H and at
// most the constants' s_max; the low byte of the result is x's centered
// residue.
uint32_t centered_byte(uint32_t sc, uint32_t shift, uint32_t h_sh, uint32_t recip, uint32_t m) {
  return mad_u24(mulhi_u24((sc << shift) + h_sh, recip), 256u - m, sc);
}
uint32_t pack_low_bytes(const uint32_t r[4]) {  // two v_perm and an or
  return perm(r[1], r[0], 0x0c0c0400u) | perm(r[3], r[2], 0x04000c0cu);
}

void check_reduce32() {
  std::vector<int32_t> xs = {INT32_MIN, INT32_MIN + 1, -1, 0, 1, INT32_MAX, INT32_MAX - 1,
                             1 << 30, -(1 << 30), (1 << 30) + 128, -(1 << 30) - 128, 65535, -65536};
  Rng rng{12345};
  for (int i = 0; i < 40000; ++i) xs.push_back(static_cast<int32_t>(rng.next()));
  for (int i = 0; i < 20000; ++i) xs.push_back(static_cast<int32_t>(rng.next() % 2147483649ull) - (1 << 30));
  uint64_t checks = 0;
  for (uint32_t m = 2; m <= 256; ++m) {
    const ModulusConsts c = make_modulus_consts(m);
    // the epilogue's reduction: u = x + 2^31, s - H = dot(bytes(u), pow_lo)
    // + (off_i32 - H)
    if (c.off_i32 < c.half || c.off_i64 < c.half || c.off_u64 < c.half) fail("offset below H", m, c.off_i32, c.off_i64, c.off_u64);
    for (size_t i = 0; i + 4 <= xs.size(); i += 4) {
      uint32_t r[4];
      for (int e = 0; e < 4; ++e) {
        const uint32_t u = static_cast<uint32_t>(xs[i + e]) + 0x80000000u;
        r[e] = centered_byte(udot4(u, c.pow_lo, c.off_i32 - c.half), c.q_shift, c.half << c.q_shift, c.q_recip, m);
      }
      const uint32_t w = pack_low_bytes(r);
      for (int e = 0; e < 4; ++e, ++checks) {
        const int64_t want = centered_ref(xs[i + e], m);
        const int8_t got = static_cast<int8_t>(w >> (8 * e));
        if (got != want) fail("reduce32", m, xs[i + e], got, want);
      }
    }
  }
  std::printf("reduce32 checks %" PRIu64 "\n", checks);
}

uint32_t pack_byte64(uint64_t u, uint32_t off, const ModulusConsts& c) {
  uint32_t s = udot4(static_cast<uint32_t>(u), c.pow_lo, off - c.half);
  s = udot4(static_cast<uint32_t>(u >> 32), c.pow_hi, s);
  return centered_byte(s, c.pq_shift, c.half << c.pq_shift, c.pq_recip, c.m);
}

void check_pack64() {
  std::vector<int64_t> xs = {INT64_MIN, INT64_MIN + 1, -1, 0, 1, INT64_MAX, INT64_MAX - 1,
                             int64_t{1} << 62, -(int64_t{1} << 62), int64_t{1} << 32, -(int64_t{1} << 32)};
  Rng rng{777};
  for (int i = 0; i < 50000; ++i) xs.push_back(static_cast<int64_t>(rng.next()));
  while (xs.size() % 4) xs.push_back(0);
  uint64_t checks = 0;
  for (uint32_t m = 2; m <= 256; ++m) {
    const ModulusConsts c = make_modulus_consts(m);
    for (size_t i = 0; i < xs.size(); i += 4) {
      uint32_t rs[4], ru[4];
      for (int e = 0; e < 4; ++e) {
        const uint64_t v = static_cast<uint64_t>(xs[i + e]);
        rs[e] = pack_byte64(v ^ 0x8000000000000000ull, c.off_i64, c);  // signed: bias 2^63
        ru[e] = pack_byte64(v, c.off_u64, c);                          // unsigned
      }
      const uint32_t ws = pack_low_bytes(rs), wu = pack_low_bytes(ru);
      for (int e = 0; e < 4; ++e, checks += 2) {
        const int64_t want_s = centered_ref(xs[i + e], m);
        const int64_t want_u = centered_ref(static_cast<__int128>(static_cast<uint64_t>(xs[i + e])), m);
        if (static_cast<int8_t>(ws >> (8 * e)) != want_s) fail("pack i64", m, xs[i + e], static_cast<int8_t>(ws >> (8 * e)), want_s);
        if (static_cast<int8_t>(wu >> (8 * e)) != want_u) fail("pack u64", m, xs[i + e], static_cast<int8_t>(wu >> (8 * e)), want_u);
      }
    }
    // finite pack: every byte value
    for (uint32_t x0 = 0; x0 < 256; x0 += 4) {
      uint32_t r[4];
      for (int e = 0; e < 4; ++e) r[e] = centered_byte(x0 + e, c.q_shift, c.half << c.q_shift, c.q_recip, m);
      const uint32_t w = pack_low_bytes(r);
      for (int e = 0; e < 4; ++e, ++checks)
        if (static_cast<int8_t>(w >> (8 * e)) != centered_ref(x0 + e, m)) fail("pack u8", m, x0 + e, 0, 0);
    }
  }
  // m = 256 planes: the kernels pack the low byte of x (pack_low_bytes), whose
  // int8 value must be the centered residue for int64 and uint64 alike
  for (size_t i = 0; i < xs.size(); i += 4) {
    uint32_t lo[4];
    for (int e = 0; e < 4; ++e) lo[e] = static_cast<uint32_t>(static_cast<uint64_t>(xs[i + e]));
    const uint32_t w = perm(lo[1], lo[0], 0x0c0c0400u) | perm(lo[3], lo[2], 0x04000c0cu);
    for (int e = 0; e < 4; ++e, checks += 2) {
      const int8_t got = static_cast<int8_t>(w >> (8 * e));
      if (got != centered_ref(xs[i + e], 256)) fail("pack i64 m=256", 256, xs[i + e], got, 0);
      if (got != centered_ref(static_cast<__int128>(static_cast<uint64_t>(xs[i + e])), 256))
        fail("pack u64 m=256", 256, xs[i + e], got, 0);
    }
  }
  std::printf("pack64 checks %" PRIu64 "\n", checks);
}

// The export kernel's digits and Horner steps (reconstruct_x) for centered
// residues r: packed digits vp and the canonical value x in 24-bit limbs.
template <uint32_t P>
void emulate_x(const int32_t* r, uint32_t (&vp)[kGarnerDigitWords], uint32_t (&x)[kWideLimbs]) {
  constexpr GarnerTable<P> T = make_garner_table<P>();
  for (uint32_t q = 0; q < kGarnerDigitWords; ++q) vp[q] = 0;
  for (uint32_t l = 0; l < kWideLimbs; ++l) x[l] = 0;
  // digits (digit 0: the raw residue byte, m_0 = 256)
  vp[0] = static_cast<uint32_t>(r[0]) & 0xFFu;
  for (uint32_t i = 1; i < P; ++i) {
    // the residue byte with its top bit flipped (r + 128) against I_i
    uint32_t s = udot4((static_cast<uint32_t>(r[i]) & 0xFFu) ^ 0x80u, T.inv[i], T.xbias[i]);
    for (uint32_t q = 0; q < (i + 3) / 4; ++q) s = udot4(vp[q], T.wpack[i][q], s);
    const uint32_t v = mad_u24(mulhi_u24(s << T.qshift[i], T.qrecip[i]), 256u - T.m[i], s) & 0xFFu;
    vp[i / 4] |= v << (8 * (i % 4));
  }
  // Horner over the active limbs of each step, limbs left unmasked between
  // steps (mad_u24 reads their low 24 bits) and masked once at the end
  x[0] = (vp[(P - 1) / 4] >> (8 * ((P - 1) % 4))) & 0xFFu;
  for (int i = static_cast<int>(P) - 2; i >= 0; --i) {
    uint32_t carry = (vp[i / 4] >> (8 * (i % 4))) & 0xFFu;
    for (uint32_t l = 0; l < T.active[i]; ++l) {
      x[l] = mad_u24(x[l], T.m[i], carry);
      carry = x[l] >> 24;
    }
    if (carry != 0) fail("horner carry out", P, i, carry, 0);
  }
  for (uint32_t l = 0; l < kWideLimbs; ++l) x[l] &= 0xFFFFFFu;
}

// Prints, for every prefix, the Garner tables and the export kernel's
// reconstruction (emulated step by step from GarnerTable<P>: digits with the
// 24-bit quotient, Horner in 24-bit limbs over the compile-time active limb
// counts, sign and magnitude) for random centered residue vectors, so the
// Python side can check them with big integers.
template <uint32_t P>
void garner_dump_p(Rng& rng) {
  constexpr GarnerTable<P> T = make_garner_table<P>();
  const GarnerConsts g = make_garner_consts(P);
  std::printf("prefix %u\n", P);
  std::printf("m");
  for (uint32_t i = 0; i < P; ++i) std::printf(" %u", g.m[i]);
  std::printf("\ninv");
  for (uint32_t i = 0; i < P; ++i) std::printf(" %u", g.inv[i]);
  std::printf("\nbias");
  for (uint32_t i = 0; i < P; ++i) std::printf(" %u", g.bias[i]);
  std::printf("\nw");
  for (uint32_t i = 0; i < P; ++i)
    for (uint32_t j = 0; j < i; ++j) std::printf(" %u", (g.wpack[i][j / 4] >> (8 * (j % 4))) & 0xFFu);
  std::printf("\nproduct");
  for (uint32_t l = 0; l < kWideLimbs; ++l) std::printf(" %u", T.product[l]);
  std::printf("\nhalf_ceil");
  for (uint32_t l = 0; l < kWideLimbs; ++l) std::printf(" %u", T.half_ceil[l]);
  std::printf("\n");
  for (int t = 0; t < 64; ++t) {
    int32_t r[kMaxPrefix];
    uint32_t vp[kGarnerDigitWords] = {};
    for (uint32_t i = 0; i < P; ++i) {
      const int32_t h = static_cast<int32_t>(T.m[i] / 2);
      r[i] = t == 0 ? -h : t == 1 ? static_cast<int32_t>(T.m[i]) - 1 - h
                                  : static_cast<int32_t>(rng.next() % T.m[i]) - h;
    }
    uint32_t x[kWideLimbs];
    emulate_x<P>(r, vp, x);
    // sign and magnitude as the kernel computes them
    uint32_t borrow = 0;
    for (uint32_t l = 0; l < kWideLimbs; ++l) borrow = (x[l] - T.half_ceil[l] - borrow) >> 31;
    const bool negative = borrow == 0;
    uint32_t d[kWideLimbs];
    borrow = 0;
    for (uint32_t l = 0; l < kWideLimbs; ++l) {
      const uint32_t u = T.product[l] - x[l] - borrow;
      borrow = u >> 31;
      d[l] = negative ? (u & 0xFFFFFFu) : x[l];
    }
    std::printf("case");
    for (uint32_t i = 0; i < P; ++i) std::printf(" %d", r[i]);
    std::printf(" |");
    for (uint32_t i = 0; i < P; ++i) std::printf(" %u", (vp[i / 4] >> (8 * (i % 4))) & 0xFFu);
    std::printf(" | %d |", negative ? 1 : 0);
    for (uint32_t l = 0; l < kWideLimbs; ++l) std::printf(" %u", d[l]);
    std::printf(" |");
    for (uint32_t l = 0; l < kWideLimbs; ++l) std::printf(" %u", x[l]);
    std::printf("\n");
  }
}

// The 64-bit export tail (value64): the low 64 bits of the centered
// (Signed) or canonical value and its admissibility under the limits
// pos / neg, as the kernel computes it. Above the digit split (int64:
// P > kSplitSigned, uint64: P > kSplitUnsigned) from the digits vp: Horner
// over the low J digits and a test of the digits from J up; otherwise from x
// in L = (P <= 9 ? 3 : 7) limbs.
template <uint32_t P>
uint64_t emulate_value64(const uint32_t (&vp)[kGarnerDigitWords], const uint32_t (&x)[kWideLimbs], bool is_signed,
                         uint64_t pos, uint64_t neg_lim, bool& ok) {
  constexpr GarnerTable<P> T = make_garner_table<P>();
  const uint32_t J = is_signed ? kSplitSigned : kSplitUnsigned;
  auto digit = [&](uint32_t i) { return (vp[i / 4] >> (8 * (i % 4))) & 0xFFu; };
  if (P > J) {
    // Horner over digits 0 .. J-1 in 3 limbs (the kernel's horner<J, 3>)
    uint32_t y[3] = {digit(J - 1), 0, 0};
    for (int i = static_cast<int>(J) - 2; i >= 0; --i) {
      uint32_t carry = digit(static_cast<uint32_t>(i));
      for (uint32_t l = 0; l < 3; ++l) {
        y[l] = mad_u24(y[l], T.m[i], carry);
        carry = y[l] >> 24;
      }
      if (carry != 0) fail("split horner carry out", P, static_cast<uint32_t>(i), carry, 0);
    }
    for (uint32_t l = 0; l < 3; ++l) y[l] &= 0xFFFFFFu;
    bool zero_top = true, max_top = true;
    for (uint32_t i = J; i < P; ++i) {
      zero_top = zero_top && digit(i) == 0;
      max_top = max_top && digit(i) == T.m[i] - 1;
    }
    const uint64_t y64 = static_cast<uint64_t>(y[0] | (y[1] << 24)) | (static_cast<uint64_t>((y[1] >> 8) | (y[2] << 16)) << 32);
    if (is_signed) {
      const uint64_t mj = ladder_product64(J);
      ok = zero_top ? y64 <= pos : (max_top && y64 > mj - 1 - neg_lim);
      return zero_top ? y64 : y64 - mj;
    }
    ok = zero_top && (y[2] >> 16) == 0 && y64 <= pos;
    return y64;
  }
  constexpr int L = P <= 9 ? 3 : 7;
  uint32_t borrow = 0;
  for (int l = 0; l < L; ++l) borrow = (x[l] - T.half_ceil[l] - borrow) >> 31;
  const bool neg = is_signed && borrow == 0;
  uint32_t v[L];
  borrow = 0;
  for (int l = 0; l < L; ++l) {
    const uint32_t t = x[l] - (neg ? T.product[l] : 0u) - borrow;
    borrow = t >> 31;
    v[l] = t & 0xFFFFFFu;
  }
  const uint64_t w = static_cast<uint64_t>(v[0] | (v[1] << 24)) | (static_cast<uint64_t>((v[1] >> 8) | (v[2] << 16)) << 32);
  const uint32_t ext = neg ? 0xFFFFFFu : 0u;
  bool fits = (v[2] >> 16) == (ext & 0xFFu);
  for (int l = 3; l < L; ++l) fits = fits && v[l] == ext;
  ok = fits && (neg ? ~w < neg_lim : w <= pos);
  return w;
}

int32_t centered_i128(__int128 v, uint32_t m) {
  __int128 r = v % static_cast<__int128>(m);
  if (r < 0) r += m;
  return static_cast<int32_t>(r >= (m + 1) / 2 ? r - m : r);
}

// Values around every 64-bit edge (0, +-2^62, +-2^63, +-2^64, +-2^65 and
// neighbours, plus random ones) within each prefix's centered / canonical
// range, through the emulated export for int64 and uint64 at several bounds;
// expected results from __int128 arithmetic.
template <uint32_t P>
void export64_p(Rng& rng, uint64_t& checks) {
  const GarnerConsts g = make_garner_consts(P);
  // prod m_i in __int128 where it fits (P <= 15: < 2^120); otherwise every
  // test value (|v| <= 2^100) is inside the range
  bool small = P <= 15;
  __int128 prod = 1;
  if (small)
    for (uint32_t i = 0; i < P; ++i) prod *= g.m[i];
  const __int128 one = 1;
  std::vector<__int128> base = {0, one << 62, (one << 63) - 1, one << 63, (one << 63) + 1, (one << 64) - 2,
                                (one << 64) - 1, one << 64, (one << 64) + 1, one << 65, (one << 72) + 5, one << 100};
  std::vector<__int128> vals;
  for (const __int128 b : base)
    for (int d = -2; d <= 2; ++d) {
      vals.push_back(b + d);
      vals.push_back(-(b + d));
    }
  for (int i = 0; i < 200; ++i) {
    const int bits = static_cast<int>(rng.next() % 70);
    __int128 v = static_cast<__int128>(rng.next() >> (64 - (bits > 63 ? 63 : bits + 1)));
    if (bits > 63) v <<= (bits - 63);
    vals.push_back(rng.next() & 1 ? -v : v);
  }
  if (small) {
    const __int128 h = (prod + 1) / 2;  // ceil(prod / 2)
    for (int d = 0; d <= 2; ++d) {
      vals.push_back(h - 1 - d);
      vals.push_back(h - prod + d);
    }
  }
  const uint64_t two63 = 1ull << 63;
  const uint64_t bounds[] = {0, 1, 1ull << 62, two63 - 1, two63, ~0ull};
  for (const __int128 v : vals) {
    for (int is_signed = 0; is_signed < 2; ++is_signed) {
      // representable: centered range [h - prod, h - 1] or canonical [0, prod)
      if (small) {
        const __int128 h = (prod + 1) / 2;
        if (is_signed ? (v < h - prod || v > h - 1) : (v < 0 || v >= prod)) continue;
      } else if (v < 0 && !is_signed) {
        continue;
      }
      int32_t r[kMaxPrefix];
      for (uint32_t i = 0; i < P; ++i) r[i] = centered_i128(v, g.m[i]);
      uint32_t vp[kGarnerDigitWords], x[kWideLimbs];
      emulate_x<P>(r, vp, x);
      for (const uint64_t b : bounds) {
        const uint64_t pos = is_signed ? (b < two63 - 1 ? b : two63 - 1) : b;
        const uint64_t neg_lim = is_signed ? (b < two63 ? b : two63) : 0;
        bool ok = false;
        const uint64_t w = emulate_value64<P>(vp, x, is_signed != 0, pos, neg_lim, ok);
        const bool want_ok = v >= 0 ? v <= static_cast<__int128>(pos) : -v <= static_cast<__int128>(neg_lim);
        const uint64_t want_w = static_cast<uint64_t>(v);
        ++checks;
        // the value written only matters for admissible results
        if (ok != want_ok || (want_ok && w != want_w)) {
          if (failures < 20)
            std::printf("export64 P=%u signed=%d v=%s%016llx%016llx bound=%llu: w %016llx ok %d, want %016llx %d\n", P,
                        is_signed, v < 0 ? "-" : "", static_cast<unsigned long long>((v < 0 ? -v : v) >> 64),
                        static_cast<unsigned long long>(v < 0 ? -v : v), static_cast<unsigned long long>(b),
                        static_cast<unsigned long long>(w), ok, static_cast<unsigned long long>(want_w), want_ok);
          ++failures;
        }
      }
    }
  }
}

template <uint32_t... Ps>
void export64_all(std::integer_sequence<uint32_t, Ps...>) {
  Rng rng{9090};
  uint64_t checks = 0;
  (export64_p<Ps + 1>(rng, checks), ...);
  std::printf("export64 checks %" PRIu64 "\n", checks);
}

template <uint32_t... Ps>
void garner_dump_all(std::integer_sequence<uint32_t, Ps...>) {
  Rng rng{4242};
  (garner_dump_p<Ps + 1>(rng), ...);
}

void garner_dump() { garner_dump_all(std::make_integer_sequence<uint32_t, kMaxPrefix>{}); }

void check_div_case(uint32_t n, uint32_t d, const DivU31& v) {
  const uint32_t got = div_u31_host(n, v);
  if (got != n / d) {
    if (++failures < 10) std::printf("div %u / %u: got %u\n", n, d, got);
  }
}

void check_div() {
  Rng rng{777};
  std::vector<uint32_t> divisors;
  for (uint32_t d = 1; d <= 5000; ++d) divisors.push_back(d);
  for (uint32_t s = 12; s < 31; ++s) {
    divisors.push_back(1u << s);
    divisors.push_back((1u << s) - 1);
    divisors.push_back((1u << s) + 1);
  }
  divisors.push_back(0x7FFFFFFFu);
  for (int i = 0; i < 2000; ++i) divisors.push_back(1u + static_cast<uint32_t>(rng.next() % 0x7FFFFFFFu));
  uint64_t cases = 0;
  for (const uint32_t d : divisors) {
    const DivU31 v = make_div_u31(d);
    if (v.shift > 31 || v.d != d || (d > 1 && v.mul <= 0x7FFFFFFFu)) ++failures;
    const uint32_t top = 0x7FFFFFFFu;
    // edges: 0, around every multiple of d near 0 and near 2^31, and random n
    for (uint32_t n = 0; n < 64; ++n) check_div_case(n, d, v);
    for (uint32_t q = 1; q < 64; ++q) {
      const uint64_t base = uint64_t{q} * d;
      if (base > top) break;
      for (int dn = -1; dn <= 1; ++dn)
        if (base + dn <= top) check_div_case(static_cast<uint32_t>(base + dn), d, v);
    }
    const uint32_t qtop = top / d;
    for (uint32_t q = qtop > 64 ? qtop - 64 : 0; q <= qtop; ++q) {
      const uint64_t base = uint64_t{q} * d;
      for (int dn = -1; dn <= 1; ++dn)
        if (base + dn <= top) check_div_case(static_cast<uint32_t>(base + dn), d, v);
    }
    for (int i = 0; i < 2000; ++i) check_div_case(static_cast<uint32_t>(rng.next() & top), d, v);
    cases += 2200;
  }
  std::printf("div checks %" PRIu64 " divisors %zu\n", cases, divisors.size());
}

}  // namespace

// ---- CRT-basis export (crt_export.hpp) ------------------------------------------

template <uint32_t P>
void crt_dump_table() {
  constexpr CrtTable<P> t = make_crt_table<P>();
  using T = CrtTable<P>;
  std::printf("table %u %u %u %u\n", P, T::kBits, T::kDigits, T::kLimbs);
  for (uint32_t i = 0; i < P; ++i) {
    std::printf("w %u", i);
    for (uint32_t c = 0; c < T::kCols; ++c) std::printf(" %d", static_cast<int>(t.w[i][c]));
    std::printf("\n");
  }
  std::printf("m16");
  for (uint32_t j = 0; j < T::kLimbs; ++j) std::printf(" %u", t.m16[j]);
  std::printf("\n");
  // the MFMA operand layout holds the same weights
  for (uint32_t l = 0; l < 64; ++l)
    for (uint32_t b = 0; b < 16; ++b) {
      const uint32_t plane = 16 * (l >> 5) + b;
      const int8_t want = plane < P ? t.w[plane][l & 31] : int8_t{0};
      const int8_t got = static_cast<int8_t>((t.frag[l][b / 4] >> (8 * (b % 4))) & 0xFFu);
      if (got != want) fail("crt fragment layout", P, l, b, got);
    }
}

template <uint32_t P>
void crt_value(const int* r) {
  constexpr CrtTable<P> t = make_crt_table<P>();
  using T = CrtTable<P>;
  int32_t s[T::kCols] = {};
  for (uint32_t c = 0; c < T::kCols; ++c)
    for (uint32_t i = 0; i < P; ++i) s[c] += r[i] * static_cast<int32_t>(t.w[i][c]);
  uint32_t limb[T::kLimbs] = {};
  int32_t sign = 0;
  crt_centered<P>(t, s, limb, sign);
  std::printf("v %u %d", P, sign);
  for (uint32_t j = 0; j < T::kLimbs; ++j) std::printf(" %u", limb[j]);
  std::printf("\n");
}

template <uint32_t... Ps>
void crt_all(std::integer_sequence<uint32_t, Ps...>) {
  (crt_dump_table<Ps + 1>(), ...);
  uint32_t p = 0;
  while (std::scanf("%u", &p) == 1) {
    int r[kMaxPrefix] = {};
    for (uint32_t i = 0; i < p && i < kMaxPrefix; ++i)
      if (std::scanf("%d", &r[i]) != 1) return;
    ((p == Ps + 1 ? (crt_value<Ps + 1>(r), 0) : 0), ...);
  }
}

// The 64-bit CRT tail (make_crt64_table, crt64_low, crt64_in_int64,
// crt64_in_uint64) at P = 9..11 against __int128 arithmetic: the centered
// value x of each test cell, its residues, the MFMA column sums of the
// table's weights, then the tail's low word and range decisions. Values:
// dense scans across every decision band (around +-2^62, +-2^63, 2^64 and
// +-M/2, in steps of one unit of the estimate and of one), and random values
// over the whole centered range.
template <uint32_t P>
void crt64_check() {
  constexpr Crt64Table<P> t = make_crt64_table<P>();
  using i128 = __int128;
  i128 M = 1;
  for (uint32_t i = 0; i < P; ++i) M *= kLadder[i];
  const i128 half = M / 2;
  const i128 two63 = static_cast<i128>(1) << 63, two64 = static_cast<i128>(1) << 64;
  long checked = 0;
  auto check = [&](i128 x) {
    if (x < -half || x >= half) return;  // centered range [-M/2, M/2)
    int32_t s[kCrt64Cols] = {};
    for (uint32_t i = 0; i < P; ++i) {
      const int m = static_cast<int>(kLadder[i]);
      int r = static_cast<int>(((x % m) + m) % m);
      if (r >= (m + 1) / 2) r -= m;
      for (uint32_t b = 0; b < kCrt64Cols; ++b) s[b] += r * t.w[i][b];
    }
    int32_t g8 = 0;
    const uint64_t lo = crt64_low<P>(t, s, g8);
    const bool in_s = crt64_in_int64<P>(t, lo, g8), want_s = x >= -two63 && x < two63;
    const i128 xc = x < 0 ? x + M : x;  // canonical
    const bool in_u = crt64_in_uint64<P>(t, lo, g8), want_u = xc < two64;
    bool bad = in_s != want_s || in_u != want_u;
    if (want_s && static_cast<int64_t>(lo) != static_cast<int64_t>(x)) bad = true;
    if (want_u && lo != static_cast<uint64_t>(xc)) bad = true;
    if (bad) {
      if (failures < 20)
        std::printf("crt64 P%u: x %.6e (hi %lld lo %llu) in_s %d/%d in_u %d/%d g8 %d\n", P, static_cast<double>(x),
                    static_cast<long long>(static_cast<int64_t>(x >> 64)), static_cast<unsigned long long>(x),
                    in_s, want_s, in_u, want_u, g8);
      ++failures;
    }
    ++checked;
  };
  // one unit of the 2^40-scaled estimate, in value terms
  const i128 unit = M >> 40;
  const i128 edges[] = {0, two63 / 2, two63, two64, -two63 / 2, -two63, -two64, half, -half};
  for (i128 e : edges) {
    for (long k = -6000; k <= 6000; ++k) check(e + k * unit);
    for (long k = -3000; k <= 3000; ++k) check(e + k);
    for (long k = -2000; k <= 2000; ++k) check(e + k * (unit / 7 + 1) + 3);
  }
  uint64_t st = 0x9E3779B97F4A7C15ull ^ P;
  auto next = [&]() {
    st += 0x9E3779B97F4A7C15ull;
    uint64_t z = st;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  };
  for (int n = 0; n < 300000; ++n) {
    const i128 r = (static_cast<i128>(next()) << 64) | next();
    const i128 mag = r & ((static_cast<i128>(1) << 100) - 1);
    check(mag % M - half);                                            // whole range
    check(static_cast<i128>(static_cast<int64_t>(next())) >> (next() & 63));  // 64-bit values of every size
    check(two64 - (static_cast<i128>(next() >> (next() & 63))));      // just below 2^64
  }
  std::printf("crt64 P%u: %ld values\n", P, checked);
}

template <uint32_t... Ps>
void crt64_all(std::integer_sequence<uint32_t, Ps...>) {
  (crt64_check<Ps + kCrt64MinP>(), ...);
}

// crt_export_fits: every export it admits has the 32-bit quantities
// crt_export_kernel forms (the output row's byte range, the last lane's byte
// offset in it, the unit count) equal to their 64-bit values and below the
// buffer-offset limit; exports just past each limit are refused.
void check_crtgate() {
  const uint64_t span_ok = (uint64_t{1} << 31) - 1;
  int admitted = 0;
  for (uint32_t L = 1; L <= 32; ++L) {
    const int64_t edge_n = static_cast<int64_t>(((uint64_t{1} << 31) - 1) / (8u * L));  // largest n with n*8L < 2^31
    const int64_t ns[] = {1, 63, 64, 65, 4096, edge_n - 1, edge_n, edge_n + 1, 70000000, int64_t{1} << 40};
    const int64_t ms[] = {1, 2, 4096, int64_t{1} << 26, (int64_t{1} << 32) - 1, int64_t{1} << 32};
    for (int64_t n : ns)
      for (int64_t m : ms)
        for (uint64_t span : {uint64_t{4096}, span_ok, span_ok + 1}) {
          const bool fits = crt_export_fits(span, m, n, L);
          const uint64_t row_bytes = static_cast<uint64_t>(n) * 8u * L;
          const uint64_t units = static_cast<uint64_t>(m) * ((static_cast<uint64_t>(n) + 63u) / 64u);
          const bool want = span < (uint64_t{1} << 31) && row_bytes < (uint64_t{1} << 31) && units < (uint64_t{1} << 32);
          if (fits != want) {
            std::printf("crtgate: span %" PRIu64 " m %" PRId64 " n %" PRId64 " L %u: fits %d, want %d\n", span, m, n,
                        L, fits, want);
            ++failures;
            continue;
          }
          if (!fits) continue;
          ++admitted;
          // the kernel's 32-bit forms
          const uint32_t range32 = static_cast<uint32_t>(static_cast<int64_t>(n) * 8 * L);
          const int last_off = static_cast<int>(static_cast<uint32_t>(n - 1) * 8u * L);
          const uint32_t units32 = static_cast<uint32_t>(m) * static_cast<uint32_t>((n + 63) / 64);
          if (range32 != row_bytes || last_off < 0 || static_cast<uint64_t>(last_off) != row_bytes - 8u * L ||
              units32 != units || static_cast<int32_t>(range32) < 0) {
            std::printf("crtgate: 32-bit forms differ at m %" PRId64 " n %" PRId64 " L %u\n", m, n, L);
            ++failures;
          }
        }
  }
  if (crt_export_fits(4096, 1, 70000000, 8)) {
    std::printf("crtgate: m 1, n 7e7, 8 limbs admitted\n");
    ++failures;
  }
  std::printf("crtgate checks %d admitted\n", admitted);
}

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  if (!std::strcmp(argv[1], "quot")) check_quot();
  else if (!std::strcmp(argv[1], "reduce32")) check_reduce32();
  else if (!std::strcmp(argv[1], "pack64")) check_pack64();
  else if (!std::strcmp(argv[1], "garner")) garner_dump();
  else if (!std::strcmp(argv[1], "div")) check_div();
  else if (!std::strcmp(argv[1], "export64")) export64_all(std::make_integer_sequence<uint32_t, kMaxPrefix>{});
  else if (!std::strcmp(argv[1], "crt")) crt_all(std::make_integer_sequence<uint32_t, kMaxPrefix>{});
  else if (!std::strcmp(argv[1], "crtgate")) check_crtgate();
  else if (!std::strcmp(argv[1], "crt64"))
    crt64_all(std::make_integer_sequence<uint32_t, kCrt64MaxP - kCrt64MinP + 1>{});
  else return 2;
  if (failures) {
    std::printf("failures %d\n", failures);
    return 1;
  }
  std::printf("ok\n");
  return 0;
}
