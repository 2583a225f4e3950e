// Full-rate integer building blocks shared by the gfx950 kernels.
//
// gfx9 VALU runs 24-bit multiplies (v_mul_hi_u32_u24, v_mad_u32_u24) at full
// rate and 32-bit ones (v_mul_lo_u32, v_mul_hi_u32) at quarter rate, so every
// small-modulus reduction here is built from byte dot products and 24-bit
// products (the constants and their exactness proofs are in tables.hpp).
#pragma once

#include <hip/hip_runtime.h>

#include "tables.hpp"

namespace rns8x {

// hi32(lo24(x) * lo24(y)): v_mul_hi_u32_u24.
__device__ __forceinline__ uint32_t mulhi_u24(uint32_t x, uint32_t y) {
  return static_cast<uint32_t>((static_cast<uint64_t>(x & 0xFFFFFFu) * (y & 0xFFFFFFu)) >> 32);
}

// lo24(a) * lo24(b) + c (mod 2^32) as v_mad_u32_u24, b uniform. Written as
// asm because the compiler lowers the same C expression to a quarter-rate
// 32- or 64-bit multiply-add.
__device__ __forceinline__ uint32_t mad_u24(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t d;
  asm("v_mad_u32_u24 %0, %1, %2, %3" : "=v"(d) : "v"(a), "s"(b), "v"(c));
  return d;
}

// Low byte of s mod m for 0 <= s <= s_max, given the make_quot24 constants of
// s_max: q = floor(s / m), and s + q * (256 - m) is congruent to s - q * m
// (which is < m <= 256) modulo 256. The upper bytes of the result are not
// meaningful. m_comp = 256 - m.
__device__ __forceinline__ uint32_t mod_low_byte(uint32_t s, uint32_t shift, uint32_t recip, uint32_t m_comp) {
  return mad_u24(mulhi_u24(s << shift, recip), m_comp, s);
}

// For u = x + 2^31 (x an int32 sum), returns a value whose low byte is
// (x + H) mod m, H = floor(m/2): s = dot(bytes(u), 2^(8b) mod m) + off_i32 is
// congruent to x + H and at most s_max, q = floor(s / m) by the 24-bit
// quotient of tables.hpp, and s + q*(256 - m) is congruent to s - q*m modulo
// 256. m_comp = 256 - m.
__device__ __forceinline__ uint32_t residue_plus_half(uint32_t u, const ModulusConsts& mc, uint32_t m_comp) {
  return mod_low_byte(__builtin_amdgcn_udot4(u, mc.pow_lo, mc.off_i32, false), mc.q_shift, mc.q_recip, m_comp);
}

// Reads accumulator elements 4g .. 4g+3 of a 32x32 MFMA tile straight from
// their AGPRs. The asm keeps the accumulators in AGPRs through an epilogue
// (the compiler otherwise copies all of them to VGPRs at once) and, being
// volatile, keeps the reads in program order with the epilogue's stores, so
// only a few values are live at a time; four per statement leave the
// scheduler four independent chains to interleave.
typedef int v16i __attribute__((ext_vector_type(16)));
struct Acc4 {
  uint32_t v[4];
};
__device__ __forceinline__ Acc4 acc_read4(const v16i& acc, int g) {
  Acc4 r;
  asm volatile(
      "v_accvgpr_read_b32 %0, %4\n\tv_accvgpr_read_b32 %1, %5\n\t"
      "v_accvgpr_read_b32 %2, %6\n\tv_accvgpr_read_b32 %3, %7"
      : "=v"(r.v[0]), "=v"(r.v[1]), "=v"(r.v[2]), "=v"(r.v[3])
      : "a"(acc[4 * g]), "a"(acc[4 * g + 1]), "a"(acc[4 * g + 2]), "a"(acc[4 * g + 3]));
  return r;
}

// Packs (r_e - H) mod 256 for e = 0..3 into one little-endian dword, where
// r_e holds (x_e + H) mod m in its low byte (other bytes ignored): the
// centered residues as int8. half2 = H * 0x10001. v_perm_b32(s0, s1, sel)
// takes result byte k from byte sel_k of s1 (0-3) or of s0 (4-7), or 0 for
// selector 0x0c; the subtraction runs on two 16-bit lanes at once.
__device__ __forceinline__ uint32_t pack_centered(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3,
                                                  uint32_t half2) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  const u16x2 h = __builtin_bit_cast(u16x2, half2);
  const u16x2 p01 = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(r1, r0, 0x0c040c00u)) - h;
  const u16x2 p23 = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(r3, r2, 0x0c040c00u)) - h;
  return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, p23), __builtin_bit_cast(uint32_t, p01), 0x06040200u);
}

// The low bytes of r0..r3 as one little-endian dword.
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3) {
  return __builtin_amdgcn_perm(r1, r0, 0x0c0c0400u) | __builtin_amdgcn_perm(r3, r2, 0x04000c0cu);
}

}  // namespace rns8x
