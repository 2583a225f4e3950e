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
// Exit status 0 and a final "ok" line when every check passes.
#include <cinttypes>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

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
uint32_t pk_sub_u16(uint32_t a, uint32_t b) {
  const uint32_t lo = (a - b) & 0xFFFFu;
  const uint32_t hi = ((a >> 16) - (b >> 16)) & 0xFFFFu;
  return lo | (hi << 16);
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
    // 32-bit reciprocal used by the pack and export kernels: exact below 2^21
    for (uint32_t s = 0; s < (1u << 21); ++s, ++checks)
      if (umulhi(s, c.recip) != s / m) fail("quot32", m, s, umulhi(s, c.recip), s / m);
  }
  std::printf("quot checks %" PRIu64 "\n", checks);
}

// GEMM epilogue: u = x + 2^31 -> residue_plus_half -> pack_centered byte.
int8_t epilogue_byte(int32_t x, const ModulusConsts& c) {
  const uint32_t u = static_cast<uint32_t>(x) + 0x80000000u;
  const uint32_t s = udot4(u, c.pow_lo, c.off_i32);
  const uint32_t q = mulhi_u24(s << c.q_shift, c.q_recip);
  return static_cast<int8_t>(mad_u24(q, 256u - c.m, s));  // low byte (x + H) mod m, H not yet subtracted
}
uint32_t pack_centered(const uint32_t r[4], uint32_t half2) {
  const uint32_t p01 = pk_sub_u16(perm(r[1], r[0], 0x0c040c00u), half2);
  const uint32_t p23 = pk_sub_u16(perm(r[3], r[2], 0x0c040c00u), half2);
  return perm(p23, p01, 0x06040200u);
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
    const uint32_t half2 = c.half * 0x00010001u;
    for (size_t i = 0; i + 4 <= xs.size(); i += 4) {
      uint32_t r[4];
      for (int e = 0; e < 4; ++e) {
        const uint32_t u = static_cast<uint32_t>(xs[i + e]) + 0x80000000u;
        const uint32_t s = udot4(u, c.pow_lo, c.off_i32);
        const uint32_t q = mulhi_u24(s << c.q_shift, c.q_recip);
        r[e] = mad_u24(q, 256u - c.m, s);
      }
      const uint32_t w = pack_centered(r, half2);
      for (int e = 0; e < 4; ++e, ++checks) {
        const int64_t want = centered_ref(xs[i + e], m);
        const int8_t got = static_cast<int8_t>(w >> (8 * e));
        if (got != want) fail("reduce32", m, xs[i + e], got, want);
      }
    }
  }
  std::printf("reduce32 checks %" PRIu64 "\n", checks);
}

void check_pack64() {
  std::vector<int64_t> xs = {INT64_MIN, INT64_MIN + 1, -1, 0, 1, INT64_MAX, INT64_MAX - 1,
                             int64_t{1} << 62, -(int64_t{1} << 62), int64_t{1} << 32, -(int64_t{1} << 32)};
  Rng rng{777};
  for (int i = 0; i < 50000; ++i) xs.push_back(static_cast<int64_t>(rng.next()));
  uint64_t checks = 0;
  for (uint32_t m = 2; m <= 256; ++m) {
    const ModulusConsts c = make_modulus_consts(m);
    for (int64_t x : xs) {
      // signed: u = x ^ 2^63, halves of u, offset off_i64
      const uint64_t u = static_cast<uint64_t>(x) ^ 0x8000000000000000ull;
      uint32_t s = udot4(static_cast<uint32_t>(u), c.pow_lo, c.off_i64);
      s = udot4(static_cast<uint32_t>(u >> 32), c.pow_hi, s);
      if (s >= (1u << 21)) fail("pack64 range", m, x, s, 0);
      const int64_t got = static_cast<int64_t>(s - umulhi(s, c.recip) * m) - c.half;
      const int64_t want = centered_ref(x, m);
      if (got != want) fail("pack i64", m, x, got, want);
      // unsigned: the same bits read as uint64, offset off_u64
      const uint64_t v = static_cast<uint64_t>(x);
      uint32_t t = udot4(static_cast<uint32_t>(v), c.pow_lo, c.off_u64);
      t = udot4(static_cast<uint32_t>(v >> 32), c.pow_hi, t);
      const int64_t got_u = static_cast<int64_t>(t - umulhi(t, c.recip) * m) - c.half;
      const int64_t want_u = centered_ref(static_cast<__int128>(v), m);
      if (got_u != want_u) fail("pack u64", m, x, got_u, want_u);
      checks += 2;
    }
  }
  std::printf("pack64 checks %" PRIu64 "\n", checks);
}

// Prints the Garner tables and, for random centered residue vectors, the
// digits the export kernel's recurrence produces (emulated), for a big-int
// check of x = sum v_i P_i against every residue.
void garner_dump() {
  Rng rng{4242};
  for (uint32_t prefix = 1; prefix <= kMaxPrefix; ++prefix) {
    const GarnerConsts g = make_garner_consts(prefix);
    std::printf("prefix %u\n", prefix);
    std::printf("m");
    for (uint32_t i = 0; i < prefix; ++i) std::printf(" %u", g.m[i]);
    std::printf("\ninv");
    for (uint32_t i = 0; i < prefix; ++i) std::printf(" %u", g.inv[i]);
    std::printf("\nbias");
    for (uint32_t i = 0; i < prefix; ++i) std::printf(" %u", g.bias[i]);
    std::printf("\nw");
    for (uint32_t i = 0; i < prefix; ++i)
      for (uint32_t j = 0; j < i; ++j) std::printf(" %u", (g.wpack[i][j / 4] >> (8 * (j % 4))) & 0xFFu);
    std::printf("\nproduct");
    for (uint32_t l = 0; l < kWideLimbs; ++l) std::printf(" %u", g.product[l]);
    std::printf("\nhalf_ceil");
    for (uint32_t l = 0; l < kWideLimbs; ++l) std::printf(" %u", g.half_ceil[l]);
    std::printf("\n");
    for (int t = 0; t < 64; ++t) {
      int32_t r[kMaxPrefix];
      uint32_t v[kMaxPrefix] = {};
      uint32_t vp[kGarnerDigitWords] = {};
      for (uint32_t i = 0; i < prefix; ++i) {
        const int32_t h = static_cast<int32_t>(g.m[i] / 2);
        // extremes first, then random centered residues
        r[i] = t == 0 ? -h : t == 1 ? static_cast<int32_t>(g.m[i]) - 1 - h
                                    : static_cast<int32_t>(rng.next() % g.m[i]) - h;
        uint32_t s = static_cast<uint32_t>(r[i] * static_cast<int32_t>(g.inv[i]) + static_cast<int32_t>(g.bias[i]));
        for (uint32_t q = 0; q < (i + 3) / 4; ++q) s = udot4(vp[q], g.wpack[i][q], s);
        if (s >= (1u << 21)) fail("garner range", g.m[i], s, i, prefix);
        v[i] = s - umulhi(s, g.recip[i]) * g.m[i];
        vp[i / 4] |= v[i] << (8 * (i % 4));
      }
      std::printf("case");
      for (uint32_t i = 0; i < prefix; ++i) std::printf(" %d", r[i]);
      std::printf(" |");
      for (uint32_t i = 0; i < prefix; ++i) std::printf(" %u", v[i]);
      std::printf("\n");
    }
  }
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  if (!std::strcmp(argv[1], "quot")) check_quot();
  else if (!std::strcmp(argv[1], "reduce32")) check_reduce32();
  else if (!std::strcmp(argv[1], "pack64")) check_pack64();
  else if (!std::strcmp(argv[1], "garner")) garner_dump();
  else return 2;
  if (failures) {
    std::printf("failures %d\n", failures);
    return 1;
  }
  std::printf("ok\n");
  return 0;
}
