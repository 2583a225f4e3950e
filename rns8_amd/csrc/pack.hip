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
// (measured 10% faster at 4096 x 4096, 9 planes). A plane with m = 256 needs
// no arithmetic: its centered residue is the low byte of x read as int8.
//
// Residue of a 64-bit value without 64-bit division (tables.hpp): split u into
// bytes, s = dot(lo bytes, 2^(8b) mod m) + dot(hi bytes, 2^(32+8b) mod m) + off
// with two v_dot4_u32_u8 (s < 2^19), then the full-rate 24-bit quotient.
// Signed inputs are biased by 2^63 (flip the top bit) and the bias is folded
// into `off`, so int64 and uint64 share the same arithmetic.
#include <type_traits>

#include "int_ops.hpp"
#include "kernels.hpp"

namespace rns8x {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef unsigned long long v2u64 __attribute__((ext_vector_type(2)));

// Largest of a block's values, combined into *out by at most one atomic max,
// skipped when the running maximum already covers it. Every thread of the
// block must call it.
__device__ __forceinline__ void block_max_to(unsigned long long best, unsigned long long* out) {
  for (int offset = 32; offset > 0; offset >>= 1) {
    const unsigned long long other = __shfl_down(best, offset, 64);
    best = other > best ? other : best;
  }
  __shared__ unsigned long long part[4];
  if ((threadIdx.x & 63u) == 0u) part[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < 4; ++w) best = part[w] > best ? part[w] : best;
    best = part[0] > best ? part[0] : best;
    if (best != 0 && __hip_atomic_load(out, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < best) atomicMax(out, best);
  }
}

// Grid-stride over 8-column chunks with 32-bit indices (the launchers reject
// matrices with 2^32 chunks or more). With kMax the kernel also proves the
// operand's magnitude for exact-wide matrices: max |x| over the valid
// elements goes to *a.max_out (zero on entry), from the same loads. With
// kStream the plane stores are non-temporal (see kStreamPackBytes).
template <bool Signed, bool Vec, bool kMax, bool kStream>
__global__ __launch_bounds__(256) void pack_native_kernel(PackArgs a, PlaneConsts pc, uint32_t chunks_per_row,
                                                          uint32_t total_chunks) {
  constexpr int kCols = 8;
  const uint64_t* const src = static_cast<const uint64_t*>(a.src);
  unsigned long long best = 0;  // kMax: largest |x| this thread has seen
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
    if constexpr (kMax) {
      // padding columns read as 0 and do not change the maximum
#pragma unroll
      for (int e = 0; e < kCols; ++e) {
        const unsigned long long x = (static_cast<unsigned long long>(hi[e]) << 32) | lo[e];
        // |INT64_MIN| = 2^63 is representable as an unsigned magnitude
        const unsigned long long mag = (Signed && static_cast<int64_t>(x) < 0) ? 0ull - x : x;
        best = mag > best ? mag : best;
      }
    }
    // When every element of the wave fits 32 bits (int32 for signed input,
    // uint32 for unsigned), one byte dot product per residue covers it: u =
    // x + 2^31 (signed) or x (unsigned) against the int32 reduction
    // constants, whose s_max covers both offsets (off_u64 = H <= off_i32).
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
    int8_t* const out = a.planes + static_cast<int64_t>(row) * a.plane_ld + c0;
    for (uint32_t p = 0; p < a.nplanes; ++p) {
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
      v2i* const dst = reinterpret_cast<v2i*>(out + static_cast<int64_t>(p) * a.plane_pitch);
      if constexpr (kStream)
        __builtin_nontemporal_store(w, dst);
      else
        *dst = w;
    }
  }
  if constexpr (kMax) {
    if (blockIdx.x == 0 && threadIdx.x == 0 && a.max_clear) *a.max_clear = 0ull;
    block_max_to(best, a.max_out);
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

// Maximum |x| of a rows x cols matrix: block (x, y) scans columns
// [2048 x, 2048 x + 2048) of rows y, y + gridDim.y, ... (coalesced 8-byte
// loads, no index division), reduces in the block and issues at most one
// atomic, skipped when the running maximum already covers it.
template <bool Signed>
__global__ __launch_bounds__(256) void max_magnitude_kernel(const uint64_t* src, int64_t rows, int64_t cols,
                                                            int64_t ld, unsigned long long* out) {
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 2048;
  unsigned long long best = 0;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const uint64_t* const rp = src + r * ld;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t c = c0 + e * 256 + threadIdx.x;
      if (c < cols) {
        const uint64_t x = rp[c];
        // |INT64_MIN| = 2^63 is representable as an unsigned magnitude
        const unsigned long long mag =
            Signed ? (static_cast<int64_t>(x) < 0 ? 0ull - x : x) : static_cast<unsigned long long>(x);
        best = mag > best ? mag : best;
      }
    }
  }
  block_max_to(best, out);
}

// Proof factors of a GEMM result whose operands both carry device-resident
// maxima: out[0] = a[0], out[1] = b[0], and word 0 of the result's previous
// proof slot cleared (one thread).
__global__ void copy_proof_factors_kernel(const unsigned long long* a, const unsigned long long* b,
                                          unsigned long long* out, unsigned long long* clear) {
  out[0] = a[0];
  out[1] = b[0];
  clear[0] = 0ull;
}

unsigned grid_for(int64_t items) {
  const int64_t blocks = (items + 255) / 256;
  return static_cast<unsigned>(blocks < 16384 ? (blocks > 0 ? blocks : 1) : 16384);
}

// Packs whose planes exceed the 256 MB Infinity Cache store them
// non-temporally. Ordinary stores leave that much dirty data in the cache,
// and its write-back then competes with the next kernel's reads: an 8192 x
// 1 x 8192 GEMV at 9 planes (604 MB of A planes, read once by an HBM-bound
// kernel) took 193 us after an ordinary pack and 142 us after a streaming
// one. Below the cache size ordinary stores win (4096^2 at 9 planes, 151 MB:
// 50 us per pack against 62 us streaming), since the cache absorbs them.
constexpr uint64_t kStreamPackBytes = uint64_t{256} << 20;

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
  auto launch_as = [&](auto sgn, auto vc, auto mx, auto st) {
    hipLaunchKernelGGL((pack_native_kernel<decltype(sgn)::value, decltype(vc)::value, decltype(mx)::value,
                                           decltype(st)::value>),
                       grid, dim3(256), 0, stream, a, consts, cpr, tot);
  };
  using T = std::true_type;
  using F = std::false_type;
  auto launch = [&](auto sgn, auto vc, auto mx) {
    if (stream_out)
      launch_as(sgn, vc, mx, T{});
    else
      launch_as(sgn, vc, mx, F{});
  };
  const bool sgn = a.kind == NativeKind::I64, mx = a.max_out != nullptr;
  if (sgn && vec && mx) launch(T{}, T{}, T{});
  else if (sgn && vec) launch(T{}, T{}, F{});
  else if (sgn && mx) launch(T{}, F{}, T{});
  else if (sgn) launch(T{}, F{}, F{});
  else if (vec && mx) launch(F{}, T{}, T{});
  else if (vec) launch(F{}, T{}, F{});
  else if (mx) launch(F{}, F{}, T{});
  else launch(F{}, F{}, F{});
  return hipGetLastError();
}

hipError_t launch_proof_factors(const unsigned long long* a, const unsigned long long* b, unsigned long long* out,
                                unsigned long long* clear, hipStream_t stream) {
  if (!a || !b || !out || !clear) return hipErrorInvalidValue;
  hipLaunchKernelGGL(copy_proof_factors_kernel, dim3(1), dim3(1), 0, stream, a, b, out, clear);
  return hipGetLastError();
}

hipError_t launch_max_magnitude(const void* src, int64_t rows, int64_t cols, int64_t ld, NativeKind kind,
                                unsigned long long* out, hipStream_t stream) {
  if (!src || !out || rows <= 0 || cols <= 0 || ld < cols) return hipErrorInvalidValue;
  // about 1024 blocks (four per CU, each scanning several rows): column
  // chunks of 2048 across x, row strides across y
  const int64_t gx = (cols + 2047) / 2048;
  if (gx > 0x7FFFFFFFll) return hipErrorInvalidValue;
  int64_t gy = 1024 / gx;
  if (gy < 1) gy = 1;
  if (gy > rows) gy = rows;
  if (gy > 65535) gy = 65535;
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  if (kind == NativeKind::I64)
    hipLaunchKernelGGL(max_magnitude_kernel<true>, grid, dim3(256), 0, stream, static_cast<const uint64_t*>(src), rows,
                       cols, ld, out);
  else
    hipLaunchKernelGGL(max_magnitude_kernel<false>, grid, dim3(256), 0, stream, static_cast<const uint64_t*>(src),
                       rows, cols, ld, out);
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
