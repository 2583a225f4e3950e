// The residue planes of 8 consecutive 64-bit elements: the inner step of
// pack.hip's native pack kernel.
//
// Residue of a 64-bit value without 64-bit division (tables.hpp): split u into
// bytes, s = dot(lo bytes, 2^(8b) mod m) + dot(hi bytes, 2^(32+8b) mod m) + off
// with two v_dot4_u32_u8 (s < 2^19), then the full-rate 24-bit quotient.
// Signed inputs are biased by 2^63 (flip the top bit) and the bias is folded
// into `off`, so int64 and uint64 share the same arithmetic. A plane with
// m = 256 needs no arithmetic: its centered residue is the low byte of x read
// as int8.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "int_ops.hpp"
#include "tables.hpp"

namespace rns8x {

// Writes the centered residues of the elements (lo[e], hi[e]) (32-bit halves;
// padding columns hold 0) for planes 0 .. nplanes-1, one aligned 8-byte run
// per plane at out + p * plane_pitch, when `store` is set. Every lane of the
// wave must call it: when every element of the wave fits 32 bits (int32 for
// signed input, uint32 for unsigned), one byte dot product per residue covers
// it (u = x + 2^31 (signed) or x (unsigned) against the int32 reduction
// constants, whose s_max covers both offsets: off_u64 = H <= off_i32).
// Lanes that do not store must hold elements that fit 32 bits (zeros do).
template <bool Signed, bool kStream>
__device__ __forceinline__ void pack_chunk8(uint32_t (&lo)[8], uint32_t (&hi)[8], int8_t* out, int64_t plane_pitch,
                                            uint32_t nplanes, const PlaneConsts& pc, bool store) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  constexpr int kCols = 8;
  bool fits = true;
#pragma unroll
  for (int e = 0; e < kCols; ++e)
    fits &= hi[e] == (Signed ? static_cast<uint32_t>(static_cast<int32_t>(lo[e]) >> 31) : 0u);
  const bool narrow = __all(fits);
  if (Signed) {
#pragma unroll
    for (int e = 0; e < kCols; ++e) {
      hi[e] ^= 0x80000000u;
      if (narrow) lo[e] ^= 0x80000000u;
    }
  }
  for (uint32_t p = 0; p < nplanes; ++p) {
    const ModulusConsts mc = pc.mod[p];
    v2i w;
    if (mc.m == 256u) {
      // x mod 256 is the low byte, and its centered value is that byte as
      // int8 (the narrow path's bias 2^31 leaves the low byte alone)
      w = v2i{static_cast<int>(pack_low_bytes(lo[0], lo[1], lo[2], lo[3])),
              static_cast<int>(pack_low_bytes(lo[4], lo[5], lo[6], lo[7]))};
    } else if (narrow) {
      // the offsets less H: the dot product gives s - H (centered_byte)
      const uint32_t off = (Signed ? mc.off_i32 : mc.off_u64) - mc.half;
      const uint32_t h_sh = in_vgpr(mc.half << mc.q_shift), m_comp = 256u - mc.m;
      uint32_t r[kCols];
#pragma unroll
      for (int e = 0; e < kCols; ++e)
        r[e] = centered_byte(__builtin_amdgcn_udot4(lo[e], mc.pow_lo, off, false), mc.q_shift, h_sh, mc.q_recip,
                             m_comp);
      w = v2i{static_cast<int>(pack_low_bytes(r[0], r[1], r[2], r[3])),
              static_cast<int>(pack_low_bytes(r[4], r[5], r[6], r[7]))};
    } else {
      const uint32_t off = (Signed ? mc.off_i64 : mc.off_u64) - mc.half;
      const uint32_t h_sh = in_vgpr(mc.half << mc.pq_shift), m_comp = 256u - mc.m;
      uint32_t r[kCols];
#pragma unroll
      for (int e = 0; e < kCols; ++e) {
        const uint32_t t = __builtin_amdgcn_udot4(lo[e], mc.pow_lo, off, false);
        r[e] = centered_byte(__builtin_amdgcn_udot4(hi[e], mc.pow_hi, t, false), mc.pq_shift, h_sh, mc.pq_recip,
                             m_comp);
      }
      w = v2i{static_cast<int>(pack_low_bytes(r[0], r[1], r[2], r[3])),
              static_cast<int>(pack_low_bytes(r[4], r[5], r[6], r[7]))};
    }
    if (store) {
      v2i* const dst = reinterpret_cast<v2i*>(out + static_cast<int64_t>(p) * plane_pitch);
      if constexpr (kStream)
        __builtin_nontemporal_store(w, dst);
      else
        *dst = w;
    }
  }
}

}  // namespace rns8x
