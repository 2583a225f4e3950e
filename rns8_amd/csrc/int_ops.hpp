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
// 32- or 64-bit multiply-add. Callers must not pass a v_dot4 result that
// the compiler's own instructions have not read first: the wait states a
// dot product's result needs are inserted only before compiler-generated
// readers.
__device__ __forceinline__ uint32_t mad_u24(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t d;
  asm("v_mad_u32_u24 %0, %1, %2, %3" : "=v"(d) : "v"(a), "s"(b), "v"(c));
  return d;
}

// A uniform value copied into a VGPR. gfx9 VALU operations read at most one
// SGPR, so (a << shift) + c with shift and c both in SGPRs compiles to a
// shift and an add; with c in a VGPR the compiler forms one
// v_lshl_add_u32. (Written with the compiler's own instructions rather than
// asm: the result of v_dot4_u32_u8 needs wait states before a dependent
// VALU read, which the compiler inserts for its instructions but not for an
// asm statement's operands.)
__device__ __forceinline__ uint32_t in_vgpr(uint32_t x) {
  uint32_t v;
  asm("v_mov_b32 %0, %1" : "=v"(v) : "s"(x));
  return v;
}

// Low byte of s mod m for 0 <= s <= s_max, given the make_quot24 constants of
// s_max: q = floor(s / m), and s + q * (256 - m) is congruent to s - q * m
// (which is < m <= 256) modulo 256. The upper bytes of the result are not
// meaningful. m_comp = 256 - m.
__device__ __forceinline__ uint32_t mod_low_byte(uint32_t s, uint32_t shift, uint32_t recip, uint32_t m_comp) {
  return mad_u24(mulhi_u24(s << shift, recip), m_comp, s);
}

// The centered residue of x modulo m as a low byte (upper bytes not
// meaningful), given sc = s - H, where s is congruent to x + H modulo m,
// 0 <= s <= s_max of the quotient constants (shift, recip), H = floor(m/2)
// and h_sh = H << shift: q = floor(s / m) comes from the 24-bit reciprocal of
// (sc << shift) + h_sh = s << shift, and sc + q*(256 - m) is congruent modulo
// 256 to s - q*m - H = ((x + H) mod m) - H, which lies in [-128, 127] and is
// the centered residue (r for r < (m+1)/2, else r - m, with r = x mod m).
// m_comp = 256 - m. Callers fold -H into the offset of the dot products that
// form s, so the subtraction costs nothing.
__device__ __forceinline__ uint32_t centered_byte(uint32_t sc, uint32_t shift, uint32_t h_sh, uint32_t recip,
                                                  uint32_t m_comp) {
  return mad_u24(mulhi_u24((sc << shift) + h_sh, recip), m_comp, sc);
}

// Per-modulus constants of the int32 reduction below: off_c = off_i32 - H
// (off_i32 >= H) and h_sh = H << q_shift.
struct CenteredI32 {
  uint32_t off_c, h_sh, m_comp;
};
__device__ __forceinline__ CenteredI32 centered_i32_consts(const ModulusConsts& mc) {
  return CenteredI32{mc.off_i32 - mc.half, in_vgpr(mc.half << mc.q_shift), 256u - mc.m};
}

// For u = x + 2^31 (x an int32 sum), the centered residue of x modulo m in
// the low byte: s = dot(bytes(u), 2^(8b) mod m) + off_i32 is congruent to
// x + H and at most s_max (tables.hpp).
__device__ __forceinline__ uint32_t centered_residue_i32(uint32_t u, const ModulusConsts& mc, const CenteredI32& k) {
  return centered_byte(__builtin_amdgcn_udot4(u, mc.pow_lo, k.off_c, false), mc.q_shift, k.h_sh, mc.q_recip,
                       k.m_comp);
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

// The low bytes of r0..r3 as one little-endian dword.
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3) {
  return __builtin_amdgcn_perm(r1, r0, 0x0c0c0400u) | __builtin_amdgcn_perm(r3, r2, 0x04000c0cu);
}

}  // namespace rns8x
