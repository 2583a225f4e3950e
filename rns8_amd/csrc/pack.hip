// Pack kernels: native operands -> modulus-major centered int8 residue planes.
//
// Reference semantics: src/cpu/cpu_reference.cpp:53-130 (res[p][r][c] =
// centered(src[r*ld + c] mod m_p), threshold (m+1)/2).
//
// HBM-bound design: each thread owns 8 consecutive columns of one row, reads
// the 64-bit inputs once and writes one aligned 8-byte run per plane, so the
// input is read a single time for all planes (the reference's large-matrix
// path re-reads it once per plane, hip_backend_pack.inc:44-58). Eight columns
// per thread (rather than 16) halve each thread's VALU chain, which lets the
// residue arithmetic of some waves overlap the memory traffic of others
// (measured 10% faster at 4096 x 4096, 9 planes). The residue arithmetic is
// pack_chunk.hpp's.
#include <type_traits>

#include "int_ops.hpp"
#include "kernels.hpp"
#include "pack_chunk.hpp"

namespace rns8x {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned long long v2u64 __attribute__((ext_vector_type(2)));

// Grid-stride over 8-column chunks with 32-bit indices (the launchers reject
// matrices with 2^32 chunks or more). With kStream the plane stores are
// non-temporal (see kStreamPackBytes).
template <bool Signed, bool Vec, bool kStream>
__global__ __launch_bounds__(256) void pack_native_kernel(PackArgs a, PlaneConsts pc, uint32_t chunks_per_row,
                                                          uint32_t total_chunks) {
  constexpr int kCols = 8;
  const uint64_t* const src = static_cast<const uint64_t*>(a.src);
  for (uint32_t ch = blockIdx.x * blockDim.x + threadIdx.x; ch < total_chunks; ch += gridDim.x * blockDim.x) {
    const uint32_t row = ch / chunks_per_row;
    const int64_t c0 = static_cast<int64_t>(ch - row * chunks_per_row) * kCols;
    const uint64_t* const rp = src + static_cast<int64_t>(row) * a.ld;
    uint32_t lo[kCols], hi[kCols];
    if (Vec && c0 + kCols <= a.cols) {
      // row start is 16-byte aligned (checked by the launcher) and c0 is even
#pragma unroll
      for (int e = 0; e < kCols; e += 2) {
        const v2u64 v = *reinterpret_cast<const v2u64*>(rp + c0 + e);
        lo[e] = static_cast<uint32_t>(v[0]);
        hi[e] = static_cast<uint32_t>(v[0] >> 32);
        lo[e + 1] = static_cast<uint32_t>(v[1]);
        hi[e + 1] = static_cast<uint32_t>(v[1] >> 32);
      }
    } else {
#pragma unroll
      for (int e = 0; e < kCols; ++e) {
        const uint64_t x = (c0 + e < a.cols) ? rp[c0 + e] : 0ull;  // padding packs as 0
        lo[e] = static_cast<uint32_t>(x);
        hi[e] = static_cast<uint32_t>(x >> 32);
      }
    }
    pack_chunk8<Signed, kStream>(lo, hi, a.planes + static_cast<int64_t>(row) * a.plane_ld + c0, a.plane_pitch,
                                 a.nplanes, pc, true);
  }
}

// Finite u8: x < 256, s = x + H < 2^9 is inside the range of the int32
// reduction constants (their s_max is at least 255 + H), and x itself is
// s - H (centered_byte).
__global__ __launch_bounds__(256) void pack_u8_kernel(PackU8Args a, ModulusConsts mc, uint32_t chunks_per_row,
                                                      uint32_t total_chunks, uint32_t vec_load) {
  const uint32_t m_comp = 256u - mc.m;
  const uint32_t h_sh = in_vgpr(mc.half << mc.q_shift);
  for (uint32_t ch = blockIdx.x * blockDim.x + threadIdx.x; ch < total_chunks; ch += gridDim.x * blockDim.x) {
    const uint32_t row = ch / chunks_per_row;
    const int64_t c0 = static_cast<int64_t>(ch - row * chunks_per_row) * 16;
    const uint8_t* const rp = a.src + static_cast<int64_t>(row) * a.ld;
    uint32_t x[16];
    if (vec_load && c0 + 16 <= a.cols) {
      // whole aligned 16-byte segment: one load
      const v4i w = *reinterpret_cast<const v4i*>(rp + c0);
#pragma unroll
      for (int e = 0; e < 16; ++e) x[e] = (static_cast<uint32_t>(w[e >> 2]) >> (8 * (e & 3))) & 0xFFu;
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) x[e] = (c0 + e < a.cols) ? rp[c0 + e] : 0u;
    }
    uint32_t r[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) r[e] = centered_byte(x[e], mc.q_shift, h_sh, mc.q_recip, m_comp);
    const v4i w = {static_cast<int>(pack_low_bytes(r[0], r[1], r[2], r[3])),
                   static_cast<int>(pack_low_bytes(r[4], r[5], r[6], r[7])),
                   static_cast<int>(pack_low_bytes(r[8], r[9], r[10], r[11])),
                   static_cast<int>(pack_low_bytes(r[12], r[13], r[14], r[15]))};
    *reinterpret_cast<v4i*>(a.plane + static_cast<int64_t>(row) * a.plane_ld + c0) = w;
  }
}

// Packs whose planes exceed the 256 MB Infinity Cache store them
// non-temporally. Ordinary stores leave that much dirty data in the cache,
// and its write-back then competes with the next kernel's reads: an 8192 x
// 1 x 8192 GEMV at 9 planes (604 MB of A planes, read once by an HBM-bound
// kernel) took 193 us after an ordinary pack and 142 us after a streaming
// one. Below the cache size ordinary stores win (4096^2 at 9 planes, 151 MB:
// 50 us per pack against 62 us streaming), since the cache absorbs them.
constexpr uint64_t kStreamPackBytes = uint64_t{256} << 20;

unsigned grid_for(int64_t items) {
  const int64_t blocks = (items + 255) / 256;
  return static_cast<unsigned>(blocks < 16384 ? (blocks > 0 ? blocks : 1) : 16384);
}

}  // namespace

hipError_t launch_pack_native(const PackArgs& a, const PlaneConsts& consts, hipStream_t stream) {
  if (!pack_args_ok(a)) return hipErrorInvalidValue;
  const int64_t chunks_per_row = a.plane_ld / 8;
  const int64_t total = chunks_per_row * a.rows;
  const bool vec = (reinterpret_cast<uintptr_t>(a.src) & 15u) == 0 && (a.ld % 2) == 0;
  const dim3 grid(grid_for(total));
  const uint32_t cpr = static_cast<uint32_t>(chunks_per_row), tot = static_cast<uint32_t>(total);
  const bool stream_out = static_cast<uint64_t>(a.nplanes) * static_cast<uint64_t>(a.rows * a.plane_ld) >=
                          kStreamPackBytes;
  auto launch_as = [&](auto sgn, auto vc, auto st) {
    hipLaunchKernelGGL((pack_native_kernel<decltype(sgn)::value, decltype(vc)::value, decltype(st)::value>), grid,
                       dim3(256), 0, stream, a, consts, cpr, tot);
  };
  using T = std::true_type;
  using F = std::false_type;
  auto launch = [&](auto sgn, auto vc) {
    if (stream_out)
      launch_as(sgn, vc, T{});
    else
      launch_as(sgn, vc, F{});
  };
  const bool sgn = a.kind == NativeKind::I64;
  if (sgn && vec) launch(T{}, T{});
  else if (sgn) launch(T{}, F{});
  else if (vec) launch(F{}, T{});
  else launch(F{}, F{});
  return hipGetLastError();
}

hipError_t launch_pack_u8(const PackU8Args& a, hipStream_t stream) {
  if (!pack_u8_args_ok(a)) return hipErrorInvalidValue;
  const int64_t chunks_per_row = a.plane_ld / 16;
  const int64_t total = chunks_per_row * a.rows;
  const uint32_t vec = (reinterpret_cast<uintptr_t>(a.src) % 16 == 0 && a.ld % 16 == 0) ? 1u : 0u;
  hipLaunchKernelGGL(pack_u8_kernel, dim3(grid_for(total)), dim3(256), 0, stream, a, make_modulus_consts(a.modulus),
                     static_cast<uint32_t>(chunks_per_row), static_cast<uint32_t>(total), vec);
  return hipGetLastError();
}

}  // namespace rns8x
