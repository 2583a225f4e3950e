// Export kernels: resident residue planes -> native integers.
//
// Reference semantics: src/reconstruct/crt.cpp:54-170 (Garner reconstruction,
// centered representative x - P for x >= ceil(P/2), bounded int64/uint64
// checks, fixed-width limb export) and src/cpu/cpu_reference.cpp:132-153
// (finite u8 canonical export).
//
// Per cell: P residue bytes -> mixed-radix digits with one exact reduction
// per digit -> integer by Horner's rule in 24-bit limbs -> sign/range
// decisions as limb comparisons -> native output. The kernels are
// instantiated per prefix P, so the Garner tables are compile-time constants
// (evaluated from the modulus ladder) and every loop over digits and limbs is
// fully unrolled with exactly the limbs each Horner step can occupy. Each
// thread handles 4 consecutive cells of a row, so every plane contributes one
// dword load; a 2-D grid (column groups x rows) needs no index division.
#include <algorithm>
#include <utility>

#include "crt_export.hpp"
#include "dma.hpp"
#include "int_ops.hpp"
#include "kernels.hpp"

namespace rns8x {
namespace {

struct ExportLimits {
  uint32_t lim_pos[kWideLimbs];  // largest admissible magnitude for a non-negative result
  uint32_t lim_neg[kWideLimbs];  // largest admissible magnitude for a negative result
  uint64_t pos64, neg64;         // the same two limits for the 64-bit kinds (neg64 <= 2^63)
  uint32_t check;                // 0: every representable value is admissible
};

// ---- arithmetic helpers ---------------------------------------------------------

// Byte 0 of `byte_src` inserted at byte k of `word` (v_perm_b32: selector
// 0-3 picks bytes of the second operand, 4-7 of the first).
template <int K>
__device__ __forceinline__ uint32_t insert_byte(uint32_t word, uint32_t byte_src) {
  constexpr uint32_t sel = (K == 0 ? 0x03020104u : K == 1 ? 0x03020400u : K == 2 ? 0x03040100u : 0x04020100u);
  return __builtin_amdgcn_perm(byte_src, word, sel);
}

// a <= b for L-limb a against a kWideLimbs-limb b (b's upper limbs nonzero
// means b exceeds every L-limb value).
template <int L>
__device__ __forceinline__ bool limbs_le(const uint32_t (&a)[L], const uint32_t* b) {
  uint32_t upper = 0;
#pragma unroll
  for (int l = L; l < static_cast<int>(kWideLimbs); ++l) upper |= b[l];
  if (upper != 0) return true;
  uint32_t borrow = 0;
#pragma unroll
  for (int l = 0; l < L; ++l) borrow = (b[l] - a[l] - borrow) >> 31;
  return borrow == 0;
}

// One cell's mixed-radix (Garner) digits v_0 .. v_{P-1}, packed 4 per dword,
// from its centered residue bytes r_i (byte E of words[i]); flipped[i] is
// words[i] ^ 0x80808080 (each byte + 128, as unsigned bytes).
template <uint32_t P, int E>
__device__ __forceinline__ void garner_digits(const uint32_t (&words)[P], const uint32_t (&flipped)[P],
                                              uint32_t (&vp)[GarnerTable<P>::kWords]) {
  constexpr GarnerTable<P> T = make_garner_table<P>();
  static_assert(T.m[0] == 256, "digit 0 is the raw residue byte only for modulus 256");
  constexpr uint32_t W = GarnerTable<P>::kWords;
#pragma unroll
  for (uint32_t q = 0; q < W; ++q) vp[q] = 0u;
  // m_0 = 256: v_0 = r_0 mod 256 is the residue byte itself
  vp[0] = (words[0] >> (8 * E)) & 0xFFu;
#pragma unroll
  for (uint32_t i = 1; i < P; ++i) {
    // (r_i + 128) * I_i + xbias_i: the flipped residue byte against I_i at
    // byte E (the other cells' bytes meet zero weights)
    uint32_t s = __builtin_amdgcn_udot4(flipped[i], T.inv[i] << (8 * E), T.xbias[i], false);
#pragma unroll
    for (uint32_t q = 0; q < (i + 3) / 4; ++q) s = __builtin_amdgcn_udot4(vp[q], T.wpack[i][q], s, false);
    const uint32_t t = mod_low_byte(s, T.qshift[i], T.qrecip[i], 256u - T.m[i]);
    switch (i % 4) {
      case 0: vp[i / 4] = insert_byte<0>(vp[i / 4], t); break;
      case 1: vp[i / 4] = insert_byte<1>(vp[i / 4], t); break;
      case 2: vp[i / 4] = insert_byte<2>(vp[i / 4], t); break;
      default: vp[i / 4] = insert_byte<3>(vp[i / 4], t); break;
    }
  }
}

// Horner over the low J digits: x = (..(v_{J-1} m_{J-2} + v_{J-2}) ..) m_0 +
// v_0 = sum_{i<J} v_i M_i in L 24-bit limbs. Limbs are kept unmasked between
// steps: v_mad_u32_u24 reads only the low 24 bits of its multiplicand, and
// the bits above are the carry already passed on, so each limb is masked
// once, at the end.
template <uint32_t J, int L, uint32_t W>
__device__ __forceinline__ void horner(const uint32_t (&vp)[W], uint32_t (&x)[L]) {
  constexpr GarnerTable<J> T = make_garner_table<J>();
#pragma unroll
  for (int l = 0; l < L; ++l) x[l] = 0u;
  x[0] = (vp[(J - 1) / 4] >> (8 * ((J - 1) % 4))) & 0xFFu;
#pragma unroll
  for (int i = static_cast<int>(J) - 2; i >= 0; --i) {
    uint32_t carry = (vp[i / 4] >> (8 * (i % 4))) & 0xFFu;
#pragma unroll
    for (int l = 0; l < L; ++l) {
      if (static_cast<uint32_t>(l) < T.active[i]) {
        x[l] = mad_u24(x[l], T.m[i], carry);
        carry = x[l] >> 24;
      }
    }
  }
#pragma unroll
  for (int l = 0; l < L; ++l) x[l] &= 0xFFFFFFu;
}

// One cell: the canonical representative x in [0, prod m_i) as L limbs.
template <uint32_t P, int L, int E>
__device__ __forceinline__ void reconstruct_x(const uint32_t (&words)[P], const uint32_t (&flipped)[P],
                                              uint32_t (&x)[L]) {
  uint32_t vp[GarnerTable<P>::kWords];
  garner_digits<P, E>(words, flipped, vp);
  horner<P, L>(vp, x);
}

// x >= ceil(P/2): the centered value is x - P (negative).
template <uint32_t P, int L>
__device__ __forceinline__ bool centered_negative(const uint32_t (&x)[L]) {
  constexpr GarnerTable<P> T = make_garner_table<P>();
  uint32_t borrow = 0;
#pragma unroll
  for (int l = 0; l < L; ++l) borrow = (x[l] - T.half_ceil[l] - borrow) >> 31;
  return borrow == 0;
}

// One cell -> sign and magnitude d (L 24-bit limbs) of the reconstructed
// value (the wide exports).
template <uint32_t P, int L, int E, bool Signed>
__device__ __forceinline__ void reconstruct(const uint32_t (&words)[P], const uint32_t (&flipped)[P], uint32_t (&d)[L],
                                            bool& negative) {
  constexpr GarnerTable<P> T = make_garner_table<P>();
  uint32_t x[L];
  reconstruct_x<P, L, E>(words, flipped, x);
  if constexpr (Signed) {
    negative = centered_negative<P, L>(x);
    uint32_t borrow = 0;
#pragma unroll
    for (int l = 0; l < L; ++l) {
      const uint32_t t = T.product[l] - x[l] - borrow;
      borrow = t >> 31;
      d[l] = negative ? (t & 0xFFFFFFu) : x[l];
    }
  } else {
    negative = false;
#pragma unroll
    for (int l = 0; l < L; ++l) d[l] = x[l];
  }
}

// x = sum_{i<J} v_i M_i (J <= 8, M_i the product of the first i ladder
// moduli) as a 64-bit integer: M_8 < 2^64. Horner's rule runs in 32 bits
// over digits 0..3 (m_0 m_1 m_2 m_3 < 2^32; v_0 + 256 v_1 are the low two
// bytes of vp[0] since m_0 = 256) and over digits 4..7 (m_4 m_5 m_6 m_7 <
// 2^32, every partial value below 2^24 as v_mad_u32_u24 needs), and one
// 32 x 32 -> 64-bit multiply-add joins the halves.
template <uint32_t J, uint32_t W>
__device__ __forceinline__ uint64_t horner64(const uint32_t (&vp)[W]) {
  static_assert(J >= 1 && J <= 8 && 4 * W >= J, "digits 0..7 of the packed words");
  static_assert(kLadder[0] == 256 && ladder_product64(4) < (uint64_t{1} << 32) &&
                    uint64_t{kLadder[4]} * kLadder[5] * kLadder[6] * kLadder[7] < (uint64_t{1} << 32) &&
                    uint64_t{kLadder[5]} * kLadder[6] * kLadder[7] < (uint64_t{1} << 24),
                "ladder bounds of the two 32-bit Horner halves");
  auto digit = [&](uint32_t i) { return (vp[i / 4] >> (8 * (i % 4))) & 0xFFu; };
  constexpr uint32_t JL = J < 4 ? J : 4;
  uint32_t lo;
  if constexpr (JL == 1) {
    lo = digit(0);
  } else if constexpr (JL == 2) {
    lo = vp[0] & 0xFFFFu;
  } else {
    uint32_t t = digit(JL - 1);
#pragma unroll
    for (int i = static_cast<int>(JL) - 2; i >= 2; --i) t = mad_u24(t, kLadder[i], digit(i));
    lo = mad_u24(t, uint32_t{kLadder[0]} * kLadder[1], vp[0] & 0xFFFFu);
  }
  if constexpr (J <= 4) {
    return lo;
  } else {
    uint32_t hi = digit(J - 1);
#pragma unroll
    for (int i = static_cast<int>(J) - 2; i >= 4; --i) hi = mad_u24(hi, kLadder[i], digit(i));
    return static_cast<uint64_t>(hi) * ladder_product64(4) + lo;
  }
}

// One cell for the 64-bit kinds: the low 64 bits of the centered (Signed) or
// canonical value v, and whether v is admissible (|v| <= bound within int64,
// resp. v <= bound within uint64; crt.cpp:113-119).
//
// Signed: an admissible result has |v| <= 2^63 < M_8, so for P > 8 its
// digits from 8 up are all 0 (v = x8 = sum_{i<8} v_i M_i) or all m_i - 1
// (v = x8 - M_8), anything else is out of range; for P <= 8 the canonical
// x < M_P < 2^64 is centered against ceil(M_P / 2). Unsigned: the canonical
// value is x8 + v_8 M_8 + ..., below 2^64 only with digits from 9 up zero and
// v_8 = 0, or v_8 = 1 and x8 < 2^64 - M_8.
template <uint32_t P, int L, int E, bool Signed>
__device__ __forceinline__ uint64_t value64(const uint32_t (&words)[P], const uint32_t (&flipped)[P],
                                            const ExportLimits& lim, bool& ok) {
  constexpr uint32_t J = P < 8 ? P : 8;
  constexpr uint64_t MJ = ladder_product64(J);
  uint32_t vp[GarnerTable<P>::kWords];
  garner_digits<P, E>(words, flipped, vp);
  const uint64_t x = horner64<J>(vp);
  if constexpr (P <= 8) {
    if constexpr (Signed) {
      // negative iff x >= ceil(M_P / 2); then |v| = M_P - x <= M_P / 2 < 2^63
      const bool neg = x >= MJ - MJ / 2;
      ok = neg ? (MJ - x <= lim.neg64) : (x <= lim.pos64);
      return neg ? x - MJ : x;
    } else {
      ok = x <= lim.pos64;
      return x;
    }
  } else if constexpr (Signed) {
    constexpr GarnerTable<P> T = make_garner_table<P>();
    bool zero_top = true, max_top = true;
#pragma unroll
    for (uint32_t i = J; i < P; ++i) {
      const uint32_t d = (vp[i / 4] >> (8 * (i % 4))) & 0xFFu;
      zero_top &= d == 0u;
      max_top &= d == T.m[i] - 1u;
    }
    // v < 0: |v| = M_8 - x, admissible iff M_8 - x <= neg64 (neg64 <= 2^63 < M_8)
    ok = zero_top ? x <= lim.pos64 : (max_top & (x >= MJ - lim.neg64));
    return zero_top ? x : x - MJ;
  } else {
    bool zero_top = true;
#pragma unroll
    for (uint32_t i = J + 1; i < P; ++i) zero_top &= ((vp[i / 4] >> (8 * (i % 4))) & 0xFFu) == 0u;
    const uint32_t v8 = vp[2] & 0xFFu;
    // v_8 <= 1 keeps the value below 2^64 when x < 2^64 - M_8 (v_8 = 1)
    const bool fits = v8 == 0u ? x <= lim.pos64 : (v8 == 1u) & (lim.pos64 >= MJ) & (x <= lim.pos64 - MJ);
    ok = zero_top & fits;
    return x + static_cast<uint64_t>(v8) * MJ;
  }
}

// Thread t takes column group t mod 2^gpr_shift of row t >> gpr_shift of the
// block's rows (narrow results fill a block with several rows; gpr_shift = 8
// is one row per block).
template <uint32_t P, int L, ExportKind Kind>
__global__ __launch_bounds__(256) void export_kernel(ExportArgs a, ExportLimits lim, uint32_t groups_per_row,
                                                     uint32_t vec_store, uint32_t gpr_shift) {
  constexpr bool kSigned = Kind == ExportKind::I64 || Kind == ExportKind::WIDE_SIGNED;
  const uint32_t gc = blockIdx.x * blockDim.x + (threadIdx.x & ((1u << gpr_shift) - 1u));
  if (gc >= groups_per_row) return;
  const int64_t c0 = static_cast<int64_t>(gc) * 4;
  const int64_t rows_per_block = static_cast<int64_t>(blockDim.x >> gpr_shift);
  bool violation = false;
  for (int64_t row = blockIdx.y * rows_per_block + (threadIdx.x >> gpr_shift); row < a.m;
       row += gridDim.y * rows_per_block) {
    const int8_t* const cell = a.c + row * a.ldc + c0;
    uint32_t words[P], flipped[P];
#pragma unroll
    for (uint32_t i = 0; i < P; ++i) {
      words[i] = *reinterpret_cast<const uint32_t*>(cell + static_cast<int64_t>(i) * a.pitch_c);
      flipped[i] = words[i] ^ 0x80808080u;
    }
    const int64_t cells = a.n - c0 < 4 ? a.n - c0 : 4;
    if constexpr (Kind == ExportKind::I64 || Kind == ExportKind::U64) {
      uint64_t w[4];
      bool ok[4];
      w[0] = value64<P, L, 0, kSigned>(words, flipped, lim, ok[0]);
      w[1] = value64<P, L, 1, kSigned>(words, flipped, lim, ok[1]);
      w[2] = value64<P, L, 2, kSigned>(words, flipped, lim, ok[2]);
      w[3] = value64<P, L, 3, kSigned>(words, flipped, lim, ok[3]);
#pragma unroll
      for (int e = 0; e < 4; ++e) violation |= (e < cells) & !ok[e];
      uint64_t* const out = static_cast<uint64_t*>(a.dst) + row * a.ld + c0;
      if (vec_store && cells == 4) {
        typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
        reinterpret_cast<u64x2*>(out)[0] = u64x2{w[0], w[1]};
        reinterpret_cast<u64x2*>(out)[1] = u64x2{w[2], w[3]};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (e < cells) out[e] = w[e];
      }
    } else {
      uint32_t d[4][L];
      bool neg[4];
      reconstruct<P, L, 0, kSigned>(words, flipped, d[0], neg[0]);
      reconstruct<P, L, 1, kSigned>(words, flipped, d[1], neg[1]);
      reconstruct<P, L, 2, kSigned>(words, flipped, d[2], neg[2]);
      reconstruct<P, L, 3, kSigned>(words, flipped, d[3], neg[3]);
      if (lim.check) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (e < cells && !limbs_le<L>(d[e], neg[e] ? lim.lim_neg : lim.lim_pos)) violation = true;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (e >= cells) continue;
        // 64-bit words of the magnitude (24-bit limb l covers bits 24l..24l+23)
        uint64_t w3[3] = {static_cast<uint64_t>(d[e][0]) | (static_cast<uint64_t>(d[e][1]) << 24) |
                              (static_cast<uint64_t>(d[e][2]) << 48),
                          static_cast<uint64_t>(d[e][2]) >> 16, 0ull};
        if constexpr (L > 3) {
          w3[1] |= (static_cast<uint64_t>(d[e][3]) << 8) | (static_cast<uint64_t>(d[e][4]) << 32) |
                   (static_cast<uint64_t>(d[e][5]) << 56);
          w3[2] = (static_cast<uint64_t>(d[e][5]) >> 8) | (static_cast<uint64_t>(d[e][6]) << 16);
        }
        uint64_t* const out = static_cast<uint64_t*>(a.dst) + (row * a.ld + c0 + e) * a.limbs;
        if (Kind == ExportKind::WIDE_SIGNED && neg[e]) {
          // two's complement of the magnitude over limbs * 64 bits
          uint64_t carry = 1;
          for (uint32_t l = 0; l < a.limbs; ++l) {
            const uint64_t s = ~(l < 3 ? w3[l] : 0ull) + carry;
            carry = (carry && s == 0) ? 1ull : 0ull;
            out[l] = s;
          }
        } else {
          for (uint32_t l = 0; l < a.limbs; ++l) out[l] = l < 3 ? w3[l] : 0ull;
        }
      }
    }
  }
  // At most one atomic per wave, and none once the flag is visible: atomics
  // on the single status word serialize (one per thread took 0.75 ms at
  // 4096 x 4096 when every cell was out of range).
  const uint64_t voters = __ballot(violation);
  if (voters != 0 && (threadIdx.x & 63u) == static_cast<uint32_t>(__ffsll(static_cast<long long>(voters)) - 1) &&
      __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u)
    atomicOr(a.status, 1u);
}

// Per-tile bounded export (reference api_export.cpp:365-410 with
// per_tile_bounds): one workgroup per (tile of this prefix group, pass of
// rows_per_pass rows); thread t takes 4 cells of row t / gpr, column group
// t % gpr, with the tile's own 64-bit limits.
template <uint32_t P, int L, ExportKind Kind>
__global__ __launch_bounds__(256) void export_tiles_kernel(ExportArgs a, const TileExport* tiles, uint32_t gpr_log2,
                                                           uint32_t rows_per_pass, uint32_t vec_store) {
  constexpr bool kSigned = Kind == ExportKind::I64;
  const TileExport t = tiles[blockIdx.x];
  const uint32_t r = blockIdx.y * rows_per_pass + (threadIdx.x >> gpr_log2);
  const uint32_t cg = threadIdx.x & ((1u << gpr_log2) - 1u);
  bool violation = false;
  if (r < t.rows && 4u * cg < t.cols) {
    const int64_t row = static_cast<int64_t>(t.row_off) + r;
    const int64_t c0 = static_cast<int64_t>(t.col_off) + 4 * cg;
    const int8_t* const cell = a.c + row * a.ldc + c0;
    uint32_t words[P], flipped[P];
#pragma unroll
    for (uint32_t i = 0; i < P; ++i) {
      words[i] = *reinterpret_cast<const uint32_t*>(cell + static_cast<int64_t>(i) * a.pitch_c);
      flipped[i] = words[i] ^ 0x80808080u;
    }
    ExportLimits lim{};
    lim.pos64 = t.pos64;
    lim.neg64 = t.neg64;
    const uint32_t cells = t.cols - 4u * cg < 4u ? t.cols - 4u * cg : 4u;
    uint64_t w[4];
    bool ok[4];
    w[0] = value64<P, L, 0, kSigned>(words, flipped, lim, ok[0]);
    w[1] = value64<P, L, 1, kSigned>(words, flipped, lim, ok[1]);
    w[2] = value64<P, L, 2, kSigned>(words, flipped, lim, ok[2]);
    w[3] = value64<P, L, 3, kSigned>(words, flipped, lim, ok[3]);
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e) violation |= (e < cells) & !ok[e];
    uint64_t* const out = static_cast<uint64_t*>(a.dst) + row * a.ld + c0;
    if (vec_store && cells == 4) {
      typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
      reinterpret_cast<u64x2*>(out)[0] = u64x2{w[0], w[1]};
      reinterpret_cast<u64x2*>(out)[1] = u64x2{w[2], w[3]};
    } else {
#pragma unroll
      for (uint32_t e = 0; e < 4; ++e)
        if (e < cells) out[e] = w[e];
    }
  }
  const uint64_t voters = __ballot(violation);
  if (voters != 0 && (threadIdx.x & 63u) == static_cast<uint32_t>(__ffsll(static_cast<long long>(voters)) - 1) &&
      __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u)
    atomicOr(a.status, 1u);
}

// Zero-output tiles: their cells are 0 (reference cpu_reference.cpp:243-246
// and the export's zero branch); same grid as export_tiles_kernel.
__global__ __launch_bounds__(256) void export_zero_tiles_kernel(ExportArgs a, const TileExport* tiles,
                                                                uint32_t gpr_log2, uint32_t rows_per_pass) {
  const TileExport t = tiles[blockIdx.x];
  const uint32_t r = blockIdx.y * rows_per_pass + (threadIdx.x >> gpr_log2);
  const uint32_t cg = threadIdx.x & ((1u << gpr_log2) - 1u);
  if (r >= t.rows || 4u * cg >= t.cols) return;
  const uint32_t cells = t.cols - 4u * cg < 4u ? t.cols - 4u * cg : 4u;
  uint64_t* const out =
      static_cast<uint64_t*>(a.dst) + (static_cast<int64_t>(t.row_off) + r) * a.ld + t.col_off + 4 * cg;
  for (uint32_t e = 0; e < cells; ++e) out[e] = 0ull;
}

typedef int v4i __attribute__((ext_vector_type(4)));

// Canonical bytes of 4 centered residues at once: a negative byte r (top bit
// set) becomes r + m, i.e. its unsigned byte plus m modulo 256; bytes are
// added without carries between them (m = 256 adds nothing).
__device__ __forceinline__ uint32_t canonical4(uint32_t w, uint32_t m4) {
  const uint32_t neg = ((w >> 7) & 0x01010101u) * 0xFFu;
  const uint32_t add = neg & m4;
  return ((w & 0x7F7F7F7Fu) + (add & 0x7F7F7F7Fu)) ^ ((w ^ add) & 0x80808080u);
}

// 16 cells per thread: one 16-byte plane load, one 16-byte store where the
// destination row segment is aligned and whole, byte stores otherwise.
__global__ __launch_bounds__(256) void export_u8_kernel(ExportU8Args a, uint32_t groups_per_row, uint32_t vec_store,
                                                        uint32_t gpr_shift) {
  const uint32_t gc = blockIdx.x * blockDim.x + (threadIdx.x & ((1u << gpr_shift) - 1u));
  if (gc >= groups_per_row) return;
  const int64_t c0 = static_cast<int64_t>(gc) * 16;
  const uint32_t m4 = (a.modulus & 0xFFu) * 0x01010101u;
  const int64_t rows_per_block = static_cast<int64_t>(blockDim.x >> gpr_shift);
  for (int64_t row = blockIdx.y * rows_per_block + (threadIdx.x >> gpr_shift); row < a.m;
       row += gridDim.y * rows_per_block) {
    const v4i w = *reinterpret_cast<const v4i*>(a.c + row * a.ldc + c0);
    const v4i out = {static_cast<int>(canonical4(static_cast<uint32_t>(w[0]), m4)),
                     static_cast<int>(canonical4(static_cast<uint32_t>(w[1]), m4)),
                     static_cast<int>(canonical4(static_cast<uint32_t>(w[2]), m4)),
                     static_cast<int>(canonical4(static_cast<uint32_t>(w[3]), m4))};
    uint8_t* const d = a.dst + row * a.ld + c0;
    if (vec_store && c0 + 16 <= a.n) {
      *reinterpret_cast<v4i*>(d) = out;
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (c0 + e < a.n) d[e] = static_cast<uint8_t>(static_cast<uint32_t>(out[e >> 2]) >> (8 * (e & 3)));
    }
  }
}

// ---- CRT-basis export on the matrix cores ----------------------------------------
//
// The reconstruction of crt_export.hpp for the exact-wide kinds: the int8
// MFMA multiplies each cell's residues (K dimension: planes, zero past P) by
// the signed base-256 digits of the CRT basis and the quotient estimate (N
// dimension: digit columns), and an integer tail turns the column sums into
// the centered value, ~115 full-rate operations per cell at any P. The
// Garner digits and Horner steps of export_kernel cost more for the wide
// kinds (every limb of the result is a multi-limb Horner chain), and less for
// the 64-bit kinds, which keep export_kernel: on MI355X at 4096 x 4096 the
// 3-limb signed export takes 180 us here against 341 us there at P = 20, and
// the 64-bit export 59 us there against 70 us here at P = 9.
//
// Per wave and iteration: 64 consecutive cells of one row. Two 16-byte DMAs
// stage planes 0..31 of those cells (zero past P, through the buffer range)
// into the wave's 2 KB of LDS as rows of 64 bytes; the 16-byte chunk c of
// plane row k sits at chunk position c ^ crt_swz(k), so the transpose reads
// below (8 rows x 16 bytes per 16-lane group) hit distinct banks. Transpose
// reads give lane l the 16 planes 16 (l >> 5) .. +15 of cell 32 jb + (l & 31)
// (the GEMM's B-fragment gather); two MFMAs (cells 0-31 and 32-63) leave
// column 8g + 4h + e of cell (l & 31) in register 4g + e of lane 32 h + (l &
// 31); one permlane32 swap per register then gives every lane all columns of
// cell l.
template <uint32_t P>
__device__ constexpr CrtTable<P> kCrt = make_crt_table<P>();

__device__ __forceinline__ uint32_t crt_swz(uint32_t k) { return (k >> 2) & 1u; }

typedef int v16i_crt __attribute__((ext_vector_type(16)));
typedef int v2i_crt __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i_crt lds_v2i_crt;
typedef unsigned v2u32_crt __attribute__((ext_vector_type(2)));

// Pipelined: each wave cycles through kDepth tiles of kDma KB (16 planes per
// KB), and the DMAs of its next kDepth - 1 units are in flight while the
// current one computes (the kernel is bound by its integer tail, and deeper
// pipelines measured no faster). Every iteration issues kDma DMAs (a DMA past the
// last unit has an empty range and lands zeros), then the cell's stores: 8 L
// bytes per lane, which the compiler may merge into as few as kStores =
// ceil(L / 2) buffer stores of at most 16 bytes. Vector memory operations
// retire in order, and after iteration i has issued its DMA the operations
// newer than unit i's DMAs are the kDepth - 1 later DMA groups and the stores
// of min(i, kDepth - 1) earlier iterations; waiting until no more than those
// are outstanding retires unit i's DMAs whether the stores were merged or not
// (unmerged ones only make the wait stricter). kL is the limb count (0: any
// count, which waits for every outstanding access).
template <uint32_t P, ExportKind Kind, uint32_t kL>
__global__ __launch_bounds__(256) void crt_export_kernel(ExportArgs a, uint32_t chunks_per_row, uint32_t units,
                                                         uint64_t plane_span) {
  using T = CrtTable<P>;
  static_assert(Kind == ExportKind::WIDE_SIGNED || Kind == ExportKind::WIDE_UNSIGNED, "exact-wide kinds only");
  constexpr uint32_t kNeeded = (T::kCols + 7) / 8 * 4;  // registers holding columns < kCols
  constexpr uint32_t kDma = P > 16 ? 2 : 1;              // 16 planes per DMA
  constexpr uint32_t kTile = 1024 * kDma;
  constexpr uint32_t kDepth = 2;
  constexpr uint32_t kStores = (kL + 1) / 2;  // fewest store instructions of 8 L bytes
  __shared__ __attribute__((aligned(16))) int8_t lds[4 * kDepth * kTile];
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int8_t* const tiles = lds + wave * kDepth * kTile;
  const uint32_t tiles_lds = lds_address(tiles);
  const v4i wfrag = *reinterpret_cast<const v4i*>(kCrt<P>.frag[lane]);
  uint32_t dma_off[kDma];
#pragma unroll
  for (uint32_t b = 0; b < kDma; ++b) {
    const uint32_t k = 16u * b + (lane >> 2);
    dma_off[b] = k < P ? k * static_cast<uint32_t>(a.pitch_c) + 16u * ((lane & 3u) ^ crt_swz(k)) : 0x80000000u;
  }
  // transpose-read addresses within a tile; with one DMA per tile the rows of
  // planes 16..31 are not held, and those lanes re-read planes 0..15 (their
  // weights are zero)
  constexpr uint32_t kRowMask = kDma == 1 ? 15u : 31u;
  const uint32_t tr_j = lane & 15u, tr_g = lane >> 4;
  uint32_t rd_lo[2], rd_hi[2];
#pragma unroll
  for (uint32_t jb = 0; jb < 2; ++jb) {
    const uint32_t ncol = 32u * jb + 16u * (tr_g & 1u) + 8u * (tr_j & 1u);
    const uint32_t k = (16u * (tr_g >> 1) + (tr_j >> 1)) & kRowMask;
    rd_lo[jb] = k * 64u + ((ncol >> 4) ^ crt_swz(k)) * 16u + (ncol & 8u);
    rd_hi[jb] = (k + 8u) * 64u + ((ncol >> 4) ^ crt_swz(k + 8u)) * 16u + (ncol & 8u);
  }
  auto issue = [&](uint32_t u, uint32_t slot) {
    const bool live = u < units;
    const uint32_t uu = live ? u : 0u;
    const uint32_t row = uu / chunks_per_row;
    const int64_t start = static_cast<int64_t>(row) * a.ldc + static_cast<int64_t>(uu - row * chunks_per_row) * 64;
    const v4i rsrc = buffer_rsrc(a.c + start, live ? static_cast<int64_t>(plane_span) - start : 0);
#pragma unroll
    for (uint32_t b = 0; b < kDma; ++b) dma16(tiles_lds + slot * kTile + 1024u * b, dma_off[b], rsrc);
  };
  const uint32_t first = blockIdx.x * 4u + wave, step = gridDim.x * 4u;
  if (first >= units) return;
  bool violation = false;
#pragma unroll
  for (uint32_t d = 0; d + 1 < kDepth; ++d) issue(first + d * step, d);
  uint32_t it = 0;
  for (uint32_t u = first; u < units; u += step, ++it) {
    const uint32_t slot = it % kDepth;
    issue(u + (kDepth - 1) * step, (it + kDepth - 1) % kDepth);
    if constexpr (kStores == 0u) {
      __builtin_amdgcn_s_waitcnt(wait_vm(0));
    } else {
      constexpr uint32_t kDmas = (kDepth - 1) * kDma;
      static_assert(kDepth == 2, "the waits below cover one earlier iteration's stores");
      if (it == 0)
        __builtin_amdgcn_s_waitcnt(wait_vm(kDmas));
      else
        __builtin_amdgcn_s_waitcnt(wait_vm(kDmas + kStores));
    }
    const int8_t* const tile = tiles + slot * kTile;
    const uint32_t row = u / chunks_per_row;
    const int64_t c0 = static_cast<int64_t>(u - row * chunks_per_row) * 64;
    v16i_crt acc[2];
#pragma unroll
    for (uint32_t jb = 0; jb < 2; ++jb) {
      const v2i_crt lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_crt*)(tile + rd_lo[jb]));
      const v2i_crt hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_crt*)(tile + rd_hi[jb]));
      acc[jb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wfrag, v4i{lo[0], lo[1], hi[0], hi[1]}, v16i_crt{}, 0, 0, 0);
    }
    // lanes 0-31 keep cell l's columns 8g+e and take its 8g+4+e from lanes
    // 32-63; lanes 32-63 the reverse for cell l
    int32_t s[32] = {};
#pragma unroll
    for (uint32_t r = 0; r < kNeeded; ++r) {
      const auto sw = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(acc[0][r]),
                                                       static_cast<uint32_t>(acc[1][r]), false, false);
      s[8 * (r / 4) + r % 4] = static_cast<int32_t>(sw[0]);
      s[8 * (r / 4) + 4 + r % 4] = static_cast<int32_t>(sw[1]);
    }
    uint32_t limb[T::kLimbs];
    int32_t sign = 0;
    crt_centered<P>(kCrt<P>, s, limb, sign);
    const int64_t col = c0 + lane;
    const bool valid = col < a.n;
    const uint32_t sg16 = static_cast<uint32_t>(sign) & 0xFFFFu;
    auto lm = [&](uint32_t j) { return j < T::kLimbs ? limb[j] : sg16; };
    // stores through a buffer over the row's n cells: lanes past n are dropped
    const uint32_t L = kL ? kL : a.limbs;
    const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(
        static_cast<uint64_t*>(a.dst) + static_cast<int64_t>(row) * a.ld * L, static_cast<short>(0),
        static_cast<int>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a.n * 8 * L))), kBufferFlags);
    const int out_off = static_cast<int>(static_cast<uint32_t>(col) * 8u * L);
    constexpr uint32_t kND = (T::kLimbs + 1) / 2;
    uint32_t d[kND];
    uint32_t fill;
    if constexpr (Kind == ExportKind::WIDE_SIGNED) {
#pragma unroll
      for (uint32_t q = 0; q < kND; ++q) d[q] = lm(2 * q) | (lm(2 * q + 1) << 16);
      fill = static_cast<uint32_t>(sign);
    } else {
      uint32_t x[T::kLimbs];
      int32_t cx = 0;
#pragma unroll
      for (uint32_t j = 0; j < T::kLimbs; ++j) {
        const int32_t t =
            static_cast<int32_t>(limb[j]) + (sign < 0 ? static_cast<int32_t>(kCrt<P>.m16[j]) : 0) + cx;
        x[j] = static_cast<uint32_t>(t) & 0xFFFFu;
        cx = t >> 16;
      }
#pragma unroll
      for (uint32_t q = 0; q < kND; ++q)
        d[q] = (2 * q < T::kLimbs ? x[2 * q] : 0u) | ((2 * q + 1 < T::kLimbs ? x[2 * q + 1] : 0u) << 16);
      fill = 0u;
    }
    // fits in L limbs: signed, every bit from 64 L - 1 up repeats the sign;
    // unsigned, every bit from 64 L up is zero
    bool fits = true;
#pragma unroll
    for (uint32_t q = 0; q < kND; ++q) {
      if (q >= 2 * L) fits &= d[q] == fill;
      if (Kind == ExportKind::WIDE_SIGNED && q + 1 == 2 * L) fits &= (d[q] >> 31) == (fill & 1u);
    }
    violation |= valid && !fits;
    auto store = [&](uint32_t l) {
      const uint32_t lo = 2 * l < kND ? d[2 * l] : fill;
      const uint32_t hi = 2 * l + 1 < kND ? d[2 * l + 1] : fill;
      __builtin_amdgcn_raw_buffer_store_b64(v2u32_crt{lo, hi}, out, out_off + static_cast<int>(8 * l), 0, 0);
    };
    if constexpr (kL != 0) {
#pragma unroll
      for (uint32_t l = 0; l < kL; ++l) store(l);
    } else {
      for (uint32_t l = 0; l < L; ++l) store(l);
    }
  }
  __builtin_amdgcn_s_waitcnt(wait_vm(0));  // no DMA outlives the wave's LDS
  const uint64_t voters = __ballot(violation);
  if (voters != 0 && lane == static_cast<uint32_t>(__ffsll(static_cast<long long>(voters)) - 1) &&
      __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u)
    atomicOr(a.status, 1u);
}

// The bounded int64 / uint64 export at P = 9..11 on the matrix cores
// (crt_export.hpp, 64-bit results): the int8 MFMA multiplies each cell's
// residues by the 14 weight columns of Crt64Table<P>, then per cell the
// 64-bit tail (the low word of X' - q M and its class) and one 8-byte store.
// Garner's digits (export_kernel) cost about 52 of its ~87 VALU instructions
// per cell at P = 9; the tail here replaces all of them.
//
// A wave handles 256 consecutive cells of a row per iteration, so each plane
// is read and the result written in runs as long as export_kernel's (64-cell
// runs measured 71 against 60 us at C3: half-line reads and 512-byte store
// runs). Three 16-byte DMAs per lane stage planes 0..11 of those cells as
// rows of 256 bytes (DMA d: planes 4d .. 4d+3, lane l: plane 4d + l / 16,
// chunk l % 16); chunk c of plane row k sits at c ^ 2 (k & 7), so the
// transpose reads hit distinct banks: a 16-lane group reads 8 plane rows of
// one chunk (8 distinct positions), and the group serviced with it reads the
// neighbouring chunk (the other parity of positions). Rows
// 12..15 are never written: their planes have zero weights. Each 64-cell
// sub-tile takes two MFMAs and leaves column 8g + 4h + e of cell (l & 31) in
// register 4g + e of lane 32 h + (l & 31); one permlane32 swap per register
// gives every lane all columns of one cell.
template <uint32_t P>
__device__ constexpr Crt64Table<P> kCrt64 = make_crt64_table<P>();

__device__ __forceinline__ uint32_t crt64_swz(uint32_t k) { return (k & 7u) << 1; }

// Grid: x = groups of four 256-cell column chunks (one per wave), y = a share
// of the rows: each wave keeps its chunk and walks rows with stride
// gridDim.y, so a row step is a few scalar additions, and the DMAs of the
// next kDepth - 1 rows are in flight while a row computes.
template <uint32_t P, ExportKind Kind>
__global__ __launch_bounds__(256) void crt64_export_kernel(ExportArgs a, ExportLimits lim, uint32_t chunks_per_row,
                                                           uint64_t plane_span) {
  static_assert(Kind == ExportKind::I64 || Kind == ExportKind::U64, "64-bit kinds only");
  static_assert(P <= 12, "three DMAs of four planes");
  constexpr uint32_t kNeeded = (kCrt64Cols + 7) / 8 * 4;  // registers holding columns < 14
  constexpr uint32_t kDma = 3;
  constexpr uint32_t kTile = 1024 * kDma;  // plane rows 0..11 of 256 bytes
  // two row slots per wave (24 KB per block, six blocks per CU); four slots
  // (three blocks per CU) measured slower
  constexpr uint32_t kDepth = 2;
  static_assert((kDepth & (kDepth - 1)) == 0 && kDepth >= 2, "slots by mask");
  __shared__ __attribute__((aligned(16))) int8_t lds[4 * kDepth * kTile];
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t chunk = blockIdx.x * 4u + wave;
  if (chunk >= chunks_per_row || static_cast<int64_t>(blockIdx.y) >= a.m) return;
  int8_t* const tiles = lds + wave * kDepth * kTile;
  const uint32_t tiles_lds = lds_address(tiles);
  const v4i wfrag = *reinterpret_cast<const v4i*>(kCrt64<P>.frag[lane]);
  uint32_t dma_off[kDma];
#pragma unroll
  for (uint32_t d = 0; d < kDma; ++d) {
    const uint32_t k = 4u * d + (lane >> 4);
    dma_off[d] = k < P ? k * static_cast<uint32_t>(a.pitch_c) + 16u * ((lane & 15u) ^ crt64_swz(k)) : 0x80000000u;
  }
  // transpose reads of sub-tile t: lanes whose planes are 16..31 re-read
  // planes 0..15, and planes 12..15 (never staged) read rows 4..7 instead:
  // all of those have zero weights
  const uint32_t tr_j = lane & 15u, tr_g = lane >> 4;
  uint32_t rd_lo[2], rd_hi[2];
#pragma unroll
  for (uint32_t jb = 0; jb < 2; ++jb) {
    const uint32_t ncol = 32u * jb + 16u * (tr_g & 1u) + 8u * (tr_j & 1u);  // within a 64-cell sub-tile
    const uint32_t k = tr_j >> 1;
    const uint32_t kh = k + 8u < 4u * kDma ? k + 8u : k;
    rd_lo[jb] = k * 256u + ((ncol >> 4) ^ crt64_swz(k)) * 16u + (ncol & 8u);
    rd_hi[jb] = kh * 256u + ((ncol >> 4) ^ crt64_swz(kh)) * 16u + (ncol & 8u);
  }
  const int64_t c0 = static_cast<int64_t>(chunk) * 256;
  const int64_t row_step = static_cast<int64_t>(gridDim.y);
  // Row cursors advance by additions: the DMAs of row dma_row read plane
  // bytes [dma_start, plane_span) (zero past it; an empty range past the last
  // row), and row `row` stores through out_row.
  const int64_t dma_step = row_step * a.ldc;
  int64_t dma_row = blockIdx.y;
  int64_t dma_start = dma_row * a.ldc + c0;
  auto issue = [&](uint32_t slot) {
    const bool live = dma_row < a.m;
    const v4i rsrc =
        buffer_rsrc(a.c + (live ? dma_start : 0), live ? static_cast<int64_t>(plane_span) - dma_start : 0);
#pragma unroll
    for (uint32_t d = 0; d < kDma; ++d) dma16(tiles_lds + slot * kTile + 1024u * d, dma_off[d], rsrc);
    dma_row += row_step;
    dma_start += dma_step;
  };
  bool violation = false;
  int64_t row = blockIdx.y;
  uint64_t* out_row = static_cast<uint64_t*>(a.dst) + row * a.ld;
  const int64_t out_step = row_step * a.ld;
  const int out_bytes = static_cast<int>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a.n * 8)));
#pragma unroll
  for (uint32_t d = 0; d + 1 < kDepth; ++d) issue(d);
  uint32_t it = 0;
  for (; row < a.m; row += row_step, out_row += out_step, ++it) {
    const uint32_t slot = it & (kDepth - 1);
    issue((it + kDepth - 1) & (kDepth - 1));
    // Vector memory operations retire in order. Issued after this row's
    // DMAs: the kDma DMAs of each of the next kDepth - 1 rows and the four
    // stores of each of min(it, kDepth - 1) earlier rows; the first rows wait
    // as if no store were outstanding (stricter).
    if (it + 1 < kDepth)
      __builtin_amdgcn_s_waitcnt(wait_vm(kDma * (kDepth - 1)));
    else
      __builtin_amdgcn_s_waitcnt(wait_vm((kDma + 4) * (kDepth - 1)));
    const int8_t* const tile = tiles + slot * kTile;
    const __amdgpu_buffer_rsrc_t out =
        __builtin_amdgcn_make_buffer_rsrc(out_row, static_cast<short>(0), out_bytes, kBufferFlags);
#pragma unroll
    for (uint32_t t = 0; t < 4; ++t) {
      v16i_crt acc[2];
#pragma unroll
      for (uint32_t jb = 0; jb < 2; ++jb) {
        // sub-tile t: chunk positions 4t .. 4t+3 (the XOR keeps them in 4t .. 4t+3 ^ 0..7)
        const v2i_crt lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_crt*)(tile + (rd_lo[jb] ^ (64u * t))));
        const v2i_crt hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_crt*)(tile + (rd_hi[jb] ^ (64u * t))));
        acc[jb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wfrag, v4i{lo[0], lo[1], hi[0], hi[1]}, v16i_crt{}, 0, 0, 0);
      }
      int32_t s[16] = {};
#pragma unroll
      for (uint32_t r = 0; r < kNeeded; ++r) {
        const auto sw = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(acc[0][r]),
                                                         static_cast<uint32_t>(acc[1][r]), false, false);
        s[8 * (r / 4) + r % 4] = static_cast<int32_t>(sw[0]);
        s[8 * (r / 4) + 4 + r % 4] = static_cast<int32_t>(sw[1]);
      }
      int32_t g8 = 0;
      const uint64_t lo = crt64_low<P>(kCrt64<P>, s, g8);
      bool ok;
      if constexpr (Kind == ExportKind::I64) {
        const bool neg = static_cast<int32_t>(lo >> 32) < 0;
        ok = crt64_in_int64<P>(kCrt64<P>, lo, g8) & (neg ? 0ull - lo <= lim.neg64 : lo <= lim.pos64);  // 0 - lo = |v|
      } else {
        ok = crt64_in_uint64<P>(kCrt64<P>, lo, g8) & (lo <= lim.pos64);
      }
      const int64_t col = c0 + 64 * t + lane;
      violation |= (col < a.n) & !ok;
      // stores through a buffer over the row's n cells: lanes past n are dropped
      __builtin_amdgcn_raw_buffer_store_b64(v2u32_crt{static_cast<uint32_t>(lo), static_cast<uint32_t>(lo >> 32)},
                                            out, static_cast<int>(static_cast<uint32_t>(col) * 8u), 0, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(wait_vm(0));  // no DMA outlives the wave's LDS
  const uint64_t voters = __ballot(violation);
  if (voters != 0 && lane == static_cast<uint32_t>(__ffsll(static_cast<long long>(voters)) - 1) &&
      __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u)
    atomicOr(a.status, 1u);
}

// Column groups x rows; rows beyond the grid's y extent are covered by the
// row loop. Rows with fewer than 256 groups share a block: 2^shift threads
// per row (shift = 8: one row per block).
uint32_t gpr_shift_for(uint32_t groups_per_row) {
  uint32_t shift = 0;
  while (shift < 8u && (1u << shift) < groups_per_row) ++shift;
  return shift;
}
dim3 grid_2d(uint32_t groups_per_row, int64_t rows) {
  const uint32_t shift = gpr_shift_for(groups_per_row);
  const uint32_t gx = (groups_per_row + 255u) / 256u;
  const int64_t per_block = int64_t{256} >> shift;
  const int64_t blocks = (rows + per_block - 1) / per_block;
  const int64_t gy = blocks < 65535 ? blocks : 65535;
  return dim3(gx, static_cast<uint32_t>(gy > 0 ? gy : 1));
}

void set_limit_u64(uint32_t (&out)[kWideLimbs], uint64_t v) { u64_to_limbs24(v, out); }

// 2^bits - 1 (bits <= 168) as 24-bit limbs
void set_limit_pow2_minus1(uint32_t (&out)[kWideLimbs], uint32_t bits) {
  for (uint32_t l = 0; l < kWideLimbs; ++l) {
    const uint32_t lo = 24u * l;
    if (bits >= lo + 24u) out[l] = 0xFFFFFFu;
    else if (bits > lo) out[l] = (1u << (bits - lo)) - 1u;
    else out[l] = 0u;
  }
}

template <uint32_t P>
hipError_t launch_export_p(const ExportArgs& a, const ExportLimits& lim, hipStream_t stream) {
  constexpr int L = P <= 9 ? 3 : 7;  // 24-bit limbs holding P: 9 moduli < 2^72, 20 < 2^168
  static_assert(make_garner_table<P>().limbs <= static_cast<uint32_t>(L), "limb count too small for P");
  const uint32_t groups_per_row = static_cast<uint32_t>(a.ldc / 4);
  const dim3 grid = grid_2d(groups_per_row, a.m);
  const uint32_t shift = gpr_shift_for(groups_per_row);
  const uint32_t vec = (reinterpret_cast<uintptr_t>(a.dst) % 16 == 0 && a.ld % 2 == 0) ? 1u : 0u;
  switch (a.kind) {
    case ExportKind::I64:
      hipLaunchKernelGGL((export_kernel<P, L, ExportKind::I64>), grid, dim3(256), 0, stream, a, lim, groups_per_row,
                         vec, shift);
      break;
    case ExportKind::U64:
      hipLaunchKernelGGL((export_kernel<P, L, ExportKind::U64>), grid, dim3(256), 0, stream, a, lim, groups_per_row,
                         vec, shift);
      break;
    case ExportKind::WIDE_SIGNED:
      hipLaunchKernelGGL((export_kernel<P, L, ExportKind::WIDE_SIGNED>), grid, dim3(256), 0, stream, a, lim,
                         groups_per_row, vec, shift);
      break;
    case ExportKind::WIDE_UNSIGNED:
      hipLaunchKernelGGL((export_kernel<P, L, ExportKind::WIDE_UNSIGNED>), grid, dim3(256), 0, stream, a, lim,
                         groups_per_row, vec, shift);
      break;
  }
  return hipGetLastError();
}

// The CRT-basis export of the exact-wide kinds, used when every plane byte it
// reads lies within 2^31 of the first plane (31-bit buffer offsets, so
// 0x80000000 marks the planes past P as out of range); export_kernel
// otherwise.
template <uint32_t P>
hipError_t launch_crt_export_p(const ExportArgs& a, uint64_t plane_span, hipStream_t stream) {
  const uint32_t chunks_per_row = static_cast<uint32_t>((a.n + 63) / 64);
  const uint32_t units = static_cast<uint32_t>(a.m) * chunks_per_row;
  const uint32_t blocks = (units + 3u) / 4u < 4096u ? (units + 3u) / 4u : 4096u;
  auto go = [&](auto kind, auto limbs) {
    hipLaunchKernelGGL((crt_export_kernel<P, decltype(kind)::value, decltype(limbs)::value>), dim3(blocks),
                       dim3(256), 0, stream, a, chunks_per_row, units, plane_span);
  };
  using K = ExportKind;
  auto wide = [&](auto kind) {
    switch (a.limbs) {
      case 1: go(kind, std::integral_constant<uint32_t, 1>{}); break;
      case 2: go(kind, std::integral_constant<uint32_t, 2>{}); break;
      case 3: go(kind, std::integral_constant<uint32_t, 3>{}); break;
      case 4: go(kind, std::integral_constant<uint32_t, 4>{}); break;
      default: go(kind, std::integral_constant<uint32_t, 0>{}); break;
    }
  };
  if (a.kind == K::WIDE_SIGNED)
    wide(std::integral_constant<K, K::WIDE_SIGNED>{});
  else if (a.kind == K::WIDE_UNSIGNED)
    wide(std::integral_constant<K, K::WIDE_UNSIGNED>{});
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

template <uint32_t P>
hipError_t launch_crt64_export_p(const ExportArgs& a, const ExportLimits& lim, uint64_t plane_span,
                                 hipStream_t stream) {
  const uint32_t chunks_per_row = static_cast<uint32_t>((a.n + 255) / 256);
  // x: groups of 4 chunks; y: toward ~8 blocks per CU in all, each wave
  // walking at least a few rows (the DMA pipeline runs along its rows)
  const uint32_t gx = (chunks_per_row + 3u) / 4u;
  const int64_t want_y = std::max<int64_t>(1, 2048 / static_cast<int64_t>(gx));
  const uint32_t gy = static_cast<uint32_t>(std::min<int64_t>({a.m, want_y, 65535}));
  if (a.kind == ExportKind::I64)
    hipLaunchKernelGGL((crt64_export_kernel<P, ExportKind::I64>), dim3(gx, gy), dim3(256), 0, stream, a, lim,
                       chunks_per_row, plane_span);
  else
    hipLaunchKernelGGL((crt64_export_kernel<P, ExportKind::U64>), dim3(gx, gy), dim3(256), 0, stream, a, lim,
                       chunks_per_row, plane_span);
  return hipGetLastError();
}

template <uint32_t... Ps>
hipError_t dispatch_crt64(uint32_t prefix, const ExportArgs& a, const ExportLimits& lim, uint64_t plane_span,
                          hipStream_t stream, std::integer_sequence<uint32_t, Ps...>) {
  hipError_t err = hipErrorInvalidValue;
  ((prefix == Ps + kCrt64MinP ? (err = launch_crt64_export_p<Ps + kCrt64MinP>(a, lim, plane_span, stream), 0) : 0),
   ...);
  return err;
}

template <uint32_t... Ps>
hipError_t dispatch_crt(uint32_t prefix, const ExportArgs& a, uint64_t plane_span, hipStream_t stream,
                        std::integer_sequence<uint32_t, Ps...>) {
  hipError_t err = hipErrorInvalidValue;
  ((prefix == Ps + 1 ? (err = launch_crt_export_p<Ps + 1>(a, plane_span, stream), 0) : 0), ...);
  return err;
}

template <uint32_t... Ps>
hipError_t dispatch_prefix(uint32_t prefix, const ExportArgs& a, const ExportLimits& lim, hipStream_t stream,
                           std::integer_sequence<uint32_t, Ps...>) {
  hipError_t err = hipErrorInvalidValue;
  ((prefix == Ps + 1 ? (err = launch_export_p<Ps + 1>(a, lim, stream), 0) : 0), ...);
  return err;
}

// Tiles of schedule edge tile_m x tile_n (powers of two, 64 .. 512): 4-cell
// column groups per tile row and the rows one 256-thread pass covers.
struct TileGrid {
  uint32_t gpr_log2, rows_per_pass;
  dim3 grid;
};
bool tile_grid(uint32_t tile_m, uint32_t tile_n, uint32_t count, TileGrid& g) {
  auto pow2 = [](uint32_t v) { return v >= 64 && v <= 512 && (v & (v - 1u)) == 0; };
  if (!pow2(tile_m) || !pow2(tile_n) || count == 0 || count > 0x7FFFFFFFu) return false;
  g.gpr_log2 = static_cast<uint32_t>(__builtin_ctz(tile_n / 4u));
  g.rows_per_pass = 256u >> g.gpr_log2;
  g.grid = dim3(count, (tile_m + g.rows_per_pass - 1) / g.rows_per_pass);
  return true;
}

bool tile_args_ok(const ExportArgs& a) {
  if (!a.c || !a.dst || a.m <= 0 || a.n <= 0 || a.ld < a.n || a.limbs != 1) return false;
  if (a.kind != ExportKind::I64 && a.kind != ExportKind::U64) return false;
  if (a.m >= (int64_t{1} << 31) || a.n >= (int64_t{1} << 31)) return false;
  if (a.ldc != padded_ld(a.n) || a.pitch_c < a.m * a.ldc || (a.pitch_c % 4) != 0) return false;
  return (reinterpret_cast<uintptr_t>(a.c) & 3u) == 0;
}

template <uint32_t P>
hipError_t launch_export_tiles_p(const ExportArgs& a, const TileExport* tiles, const TileGrid& g, hipStream_t stream) {
  constexpr int L = P <= 9 ? 3 : 7;
  const uint32_t vec = (reinterpret_cast<uintptr_t>(a.dst) % 16 == 0 && a.ld % 2 == 0) ? 1u : 0u;
  if (a.kind == ExportKind::I64)
    hipLaunchKernelGGL((export_tiles_kernel<P, L, ExportKind::I64>), g.grid, dim3(256), 0, stream, a, tiles,
                       g.gpr_log2, g.rows_per_pass, vec);
  else
    hipLaunchKernelGGL((export_tiles_kernel<P, L, ExportKind::U64>), g.grid, dim3(256), 0, stream, a, tiles,
                       g.gpr_log2, g.rows_per_pass, vec);
  return hipGetLastError();
}

template <uint32_t... Ps>
hipError_t dispatch_tiles(uint32_t prefix, const ExportArgs& a, const TileExport* tiles, const TileGrid& g,
                          hipStream_t stream, std::integer_sequence<uint32_t, Ps...>) {
  hipError_t err = hipErrorInvalidValue;
  ((prefix == Ps + 1 ? (err = launch_export_tiles_p<Ps + 1>(a, tiles, g, stream), 0) : 0), ...);
  return err;
}

}  // namespace

hipError_t launch_export_tiles(const ExportArgs& a, uint32_t prefix, const TileExport* d_tiles, uint32_t count,
                               uint32_t tile_m, uint32_t tile_n, hipStream_t stream) {
  TileGrid g;
  if (!tile_args_ok(a) || !a.status || !d_tiles || !tile_grid(tile_m, tile_n, count, g)) return hipErrorInvalidValue;
  if (prefix == 0 || prefix > kMaxPrefix) return hipErrorInvalidValue;
  return dispatch_tiles(prefix, a, d_tiles, g, stream, std::make_integer_sequence<uint32_t, kMaxPrefix>{});
}

hipError_t launch_export_zero_tiles(const ExportArgs& a, const TileExport* d_tiles, uint32_t count, uint32_t tile_m,
                                    uint32_t tile_n, hipStream_t stream) {
  TileGrid g;
  if (!tile_args_ok(a) || !d_tiles || !tile_grid(tile_m, tile_n, count, g)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(export_zero_tiles_kernel, g.grid, dim3(256), 0, stream, a, d_tiles, g.gpr_log2,
                     g.rows_per_pass);
  return hipGetLastError();
}

hipError_t launch_export(const ExportArgs& a, uint32_t prefix, hipStream_t stream) {
  if (!export_args_ok(a, prefix)) return hipErrorInvalidValue;
  ExportLimits lim{};
  lim.check = 1;
  switch (a.kind) {
    case ExportKind::I64: {
      // |v| <= bound and v in int64: magnitude <= min(bound, 2^63 - 1) for
      // v >= 0 and <= min(bound, 2^63) for v < 0 (crt.cpp:113-119).
      const uint64_t two63 = 1ull << 63;
      lim.pos64 = a.bound < two63 - 1 ? a.bound : two63 - 1;
      lim.neg64 = a.bound < two63 ? a.bound : two63;
      break;
    }
    case ExportKind::U64:
      lim.pos64 = a.bound;  // no negative results
      break;
    case ExportKind::WIDE_SIGNED:
      if (a.limbs >= 3) {
        lim.check = 0;  // 192 bits hold every centered value below 2^155
      } else {
        set_limit_pow2_minus1(lim.lim_pos, 64u * a.limbs - 1u);  // 2^(bits-1) - 1
        set_limit_pow2_minus1(lim.lim_neg, 64u * a.limbs - 1u);
        // negative magnitudes may reach 2^(bits-1): add one to the limit
        uint32_t carry = 1;
        for (uint32_t l = 0; l < kWideLimbs; ++l) {
          const uint32_t t = lim.lim_neg[l] + carry;
          lim.lim_neg[l] = t & 0xFFFFFFu;
          carry = t >> 24;
        }
      }
      break;
    case ExportKind::WIDE_UNSIGNED:
      if (a.limbs >= 3) {
        lim.check = 0;
      } else {
        set_limit_pow2_minus1(lim.lim_pos, 64u * a.limbs);
        set_limit_pow2_minus1(lim.lim_neg, 64u * a.limbs);
      }
      break;
  }
  // bytes from the first plane's start to the end of the last plane's rows
  const uint64_t plane_span = static_cast<uint64_t>(prefix - 1) * static_cast<uint64_t>(a.pitch_c) +
                              static_cast<uint64_t>(a.m) * static_cast<uint64_t>(a.ldc);
  const bool wide = a.kind == ExportKind::WIDE_SIGNED || a.kind == ExportKind::WIDE_UNSIGNED;
  const bool crt = wide && crt_export_fits(plane_span, a.m, a.n, a.limbs) &&
                   (reinterpret_cast<uintptr_t>(a.c) & 15u) == 0 && (a.pitch_c % 16) == 0;
  if (crt) return dispatch_crt(prefix, a, plane_span, stream, std::make_integer_sequence<uint32_t, kMaxPrefix>{});
  // 64-bit kinds at P = 9..11: the CRT-basis form with the 64-bit tail, for
  // results at least one 256-column chunk wide (a wave stages and multiplies
  // a whole chunk per row, so narrower results, GEMV outputs above all, run
  // the per-cell kernel: 8192 x 1 takes 4.4 us there against 12.9 us here)
  const bool crt64 = (a.kind == ExportKind::I64 || a.kind == ExportKind::U64) && prefix >= kCrt64MinP &&
                     prefix <= kCrt64MaxP && a.n >= 256 && crt_export_fits(plane_span, a.m, a.n, 1) &&
                     (reinterpret_cast<uintptr_t>(a.c) & 15u) == 0 && (a.pitch_c % 16) == 0 &&
                     (reinterpret_cast<uintptr_t>(a.dst) & 7u) == 0;
  if (crt64)
    return dispatch_crt64(prefix, a, lim, plane_span, stream,
                          std::make_integer_sequence<uint32_t, kCrt64MaxP - kCrt64MinP + 1>{});
  return dispatch_prefix(prefix, a, lim, stream, std::make_integer_sequence<uint32_t, kMaxPrefix>{});
}

hipError_t launch_export_u8(const ExportU8Args& a, hipStream_t stream) {
  if (!export_u8_args_ok(a)) return hipErrorInvalidValue;
  const uint32_t groups_per_row = static_cast<uint32_t>(a.ldc / 16);
  const uint32_t vec = (reinterpret_cast<uintptr_t>(a.dst) % 16 == 0 && a.ld % 16 == 0) ? 1u : 0u;
  hipLaunchKernelGGL(export_u8_kernel, grid_2d(groups_per_row, a.m), dim3(256), 0, stream, a, groups_per_row, vec,
                     gpr_shift_for(groups_per_row));
  return hipGetLastError();
}

}  // namespace rns8x
