// Export kernels: resident residue planes -> native integers.
//
// Reference semantics: src/reconstruct/crt.cpp:54-170 (Garner reconstruction,
// centered representative x - P for x >= ceil(P/2), bounded int64/uint64
// checks, fixed-width limb export) and src/cpu/cpu_reference.cpp:132-153
// (finite u8 canonical export).
//
// Per cell: P residue bytes -> mixed-radix digits with one exact reduction
// per digit (tables.hpp, GarnerConsts) -> integer by Horner's rule in 24-bit
// limbs -> sign/range decisions as limb comparisons against host-computed
// constants -> native output. Each thread handles 4 consecutive cells of a
// row so every plane contributes one dword load.
#include "kernels.hpp"

namespace rns8x {
namespace {

struct ExportLimits {
  uint32_t lim_pos[kWideLimbs];  // largest admissible magnitude for a non-negative result
  uint32_t lim_neg[kWideLimbs];  // largest admissible magnitude for a negative result
  uint32_t check;                // 0: every representable value is admissible
};

// a <= b where a has L 24-bit limbs and b has kWideLimbs (b's upper limbs may
// be nonzero, in which case b exceeds every L-limb value).
template <int L>
__device__ __forceinline__ bool limbs_le(const uint32_t (&a)[L], const uint32_t* b) {
  uint32_t upper = 0;
#pragma unroll
  for (int l = L; l < static_cast<int>(kWideLimbs); ++l) upper |= b[l];
  if (upper != 0) return true;
  uint32_t borrow = 0;
#pragma unroll
  for (int l = 0; l < L; ++l) {
    const uint32_t d = b[l] - a[l] - borrow;
    borrow = d >> 31;
  }
  return borrow == 0;
}

template <int L, ExportKind Kind>
__global__ __launch_bounds__(256) void export_kernel(ExportArgs a, GarnerConsts g, ExportLimits lim,
                                                     int64_t groups_per_row, int64_t total_groups) {
  const uint32_t P = g.prefix;
  for (int64_t gi = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; gi < total_groups;
       gi += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = gi / groups_per_row;
    const int64_t c0 = (gi - row * groups_per_row) * 4;
    const int8_t* const cell = a.c + row * a.ldc + c0;
    uint32_t words[kMaxPrefix];
#pragma unroll
    for (uint32_t i = 0; i < kMaxPrefix; ++i)
      words[i] = i < P ? *reinterpret_cast<const uint32_t*>(cell + static_cast<int64_t>(i) * a.pitch_c) : 0u;
    bool violation = false;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t col = c0 + e;
      // ---- mixed-radix digits ----
      uint32_t vp[kGarnerDigitWords] = {0u, 0u, 0u, 0u, 0u};
#pragma unroll
      for (uint32_t i = 0; i < kMaxPrefix; ++i) {
        if (i < P) {
          const int32_t r = static_cast<int32_t>(static_cast<int8_t>(words[i] >> (8 * e)));
          uint32_t s = static_cast<uint32_t>(r * static_cast<int32_t>(g.inv[i]) + static_cast<int32_t>(g.bias[i]));
#pragma unroll
          for (uint32_t q = 0; q < (i + 3) / 4; ++q) s = __builtin_amdgcn_udot4(vp[q], g.wpack[i][q], s, false);
          const uint32_t v = s - __umulhi(s, g.recip[i]) * g.m[i];
          vp[i / 4] |= v << (8 * (i % 4));
        }
      }
      // ---- Horner: x = (..(v_{P-1} m_{P-2} + v_{P-2}) ..) m_0 + v_0 ----
      uint32_t x[L];
#pragma unroll
      for (int l = 0; l < L; ++l) x[l] = 0u;
#pragma unroll
      for (int i = static_cast<int>(kMaxPrefix) - 1; i >= 0; --i) {
        if (static_cast<uint32_t>(i) < P) {
          const uint32_t v = (vp[i / 4] >> (8 * (i % 4))) & 0xFFu;
          const uint32_t mul = static_cast<uint32_t>(i) + 1u < P ? g.m[i] : 0u;  // top digit starts x
          uint32_t carry = v;
#pragma unroll
          for (int l = 0; l < L; ++l) {
            const uint32_t t = __umul24(x[l], mul) + carry;
            x[l] = t & 0xFFFFFFu;
            carry = t >> 24;
          }
        }
      }
      // ---- sign and magnitude ----
      bool negative = false;
      uint32_t d[L];
      if (Kind == ExportKind::I64 || Kind == ExportKind::WIDE_SIGNED) {
        uint32_t borrow = 0;
#pragma unroll
        for (int l = 0; l < L; ++l) {
          const uint32_t t = x[l] - g.half_ceil[l] - borrow;
          borrow = t >> 31;
        }
        negative = borrow == 0;  // x >= ceil(P/2)
        borrow = 0;
#pragma unroll
        for (int l = 0; l < L; ++l) {
          const uint32_t t = g.product[l] - x[l] - borrow;  // P - x when negative
          borrow = t >> 31;
          d[l] = negative ? (t & 0xFFFFFFu) : x[l];
        }
      } else {
#pragma unroll
        for (int l = 0; l < L; ++l) d[l] = x[l];
      }
      const bool in_row = col < a.n;
      if (lim.check && in_row) {
        if (!limbs_le<L>(d, negative ? lim.lim_neg : lim.lim_pos)) violation = true;
      }
      if (!in_row) continue;
      // ---- 64-bit words of the magnitude ----
      uint64_t w0 = static_cast<uint64_t>(d[0]) | (static_cast<uint64_t>(d[1]) << 24) |
                    (static_cast<uint64_t>(d[2]) << 48);
      if (Kind == ExportKind::I64) {
        static_cast<int64_t*>(a.dst)[row * a.ld + col] = static_cast<int64_t>(negative ? (0ull - w0) : w0);
      } else if (Kind == ExportKind::U64) {
        static_cast<uint64_t*>(a.dst)[row * a.ld + col] = w0;
      } else {
        // bits 64..167 of the magnitude (24-bit limb l covers bits 24l..24l+23)
        uint64_t w[3] = {w0, static_cast<uint64_t>(d[2]) >> 16, 0ull};
        if (L > 3) {
          w[1] |= (static_cast<uint64_t>(d[3]) << 8) | (static_cast<uint64_t>(d[4]) << 32) |
                  (static_cast<uint64_t>(d[5]) << 56);
          w[2] = (static_cast<uint64_t>(d[5]) >> 8) | (static_cast<uint64_t>(d[L > 6 ? 6 : 0]) << 16);
        }
        uint64_t* const out = static_cast<uint64_t*>(a.dst) + (row * a.ld + col) * a.limbs;
        if (Kind == ExportKind::WIDE_SIGNED && negative) {
          // two's complement of the magnitude over limbs*64 bits
          uint64_t carry = 1;
          for (uint32_t l = 0; l < a.limbs; ++l) {
            const uint64_t word = l < 3 ? w[l] : 0ull;
            const uint64_t inv = ~word;
            const uint64_t s = inv + carry;
            carry = (carry && s == 0) ? 1ull : 0ull;
            out[l] = s;
          }
        } else {
          for (uint32_t l = 0; l < a.limbs; ++l) out[l] = l < 3 ? w[l] : 0ull;
        }
      }
    }
    if (violation) atomicOr(a.status, 1u);
  }
}

__global__ __launch_bounds__(256) void export_u8_kernel(ExportU8Args a, int64_t groups_per_row, int64_t total) {
  for (int64_t gi = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; gi < total;
       gi += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = gi / groups_per_row;
    const int64_t c0 = (gi - row * groups_per_row) * 4;
    const uint32_t word = *reinterpret_cast<const uint32_t*>(a.c + row * a.ldc + c0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (c0 + e < a.n) {
        const int32_t r = static_cast<int32_t>(static_cast<int8_t>(word >> (8 * e)));
        a.dst[row * a.ld + c0 + e] = static_cast<uint8_t>(r < 0 ? r + static_cast<int32_t>(a.modulus) : r);
      }
    }
  }
}

unsigned grid_for(int64_t items) {
  const int64_t blocks = (items + 255) / 256;
  return static_cast<unsigned>(blocks < 16384 ? (blocks > 0 ? blocks : 1) : 16384);
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

template <int L>
hipError_t launch_export_l(const ExportArgs& a, const GarnerConsts& g, const ExportLimits& lim, hipStream_t stream) {
  const int64_t groups_per_row = a.ldc / 4;
  const int64_t total = groups_per_row * a.m;
  const dim3 grid(grid_for(total));
  switch (a.kind) {
    case ExportKind::I64:
      hipLaunchKernelGGL((export_kernel<L, ExportKind::I64>), grid, dim3(256), 0, stream, a, g, lim, groups_per_row,
                         total);
      break;
    case ExportKind::U64:
      hipLaunchKernelGGL((export_kernel<L, ExportKind::U64>), grid, dim3(256), 0, stream, a, g, lim, groups_per_row,
                         total);
      break;
    case ExportKind::WIDE_SIGNED:
      hipLaunchKernelGGL((export_kernel<L, ExportKind::WIDE_SIGNED>), grid, dim3(256), 0, stream, a, g, lim,
                         groups_per_row, total);
      break;
    case ExportKind::WIDE_UNSIGNED:
      hipLaunchKernelGGL((export_kernel<L, ExportKind::WIDE_UNSIGNED>), grid, dim3(256), 0, stream, a, g, lim,
                         groups_per_row, total);
      break;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_export(const ExportArgs& a, const GarnerConsts& g, hipStream_t stream) {
  if (!a.c || !a.dst || !a.status || a.m <= 0 || a.n <= 0 || a.ld < a.n) return hipErrorInvalidValue;
  if (g.prefix == 0 || g.prefix > kMaxPrefix) return hipErrorInvalidValue;
  if (a.ldc != padded_ld(a.n) || a.pitch_c < a.m * a.ldc || (a.pitch_c % 4) != 0) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(a.c) & 3u) != 0) return hipErrorInvalidValue;
  if (a.limbs == 0 || a.limbs > 32) return hipErrorInvalidValue;
  if ((a.kind == ExportKind::I64 || a.kind == ExportKind::U64) && a.limbs != 1) return hipErrorInvalidValue;
  ExportLimits lim{};
  lim.check = 1;
  switch (a.kind) {
    case ExportKind::I64: {
      // |v| <= bound and v in int64: magnitude <= min(bound, 2^63 - 1) for
      // v >= 0 and <= min(bound, 2^63) for v < 0 (crt.cpp:113-119).
      const uint64_t two63 = 1ull << 63;
      set_limit_u64(lim.lim_pos, a.bound < two63 - 1 ? a.bound : two63 - 1);
      set_limit_u64(lim.lim_neg, a.bound < two63 ? a.bound : two63);
      break;
    }
    case ExportKind::U64:
      set_limit_u64(lim.lim_pos, a.bound);
      set_limit_u64(lim.lim_neg, a.bound);
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
  if (g.prefix <= 9) return launch_export_l<3>(a, g, lim, stream);
  return launch_export_l<7>(a, g, lim, stream);
}

hipError_t launch_export_u8(const ExportU8Args& a, hipStream_t stream) {
  if (!a.c || !a.dst || a.m <= 0 || a.n <= 0 || a.ld < a.n) return hipErrorInvalidValue;
  if (a.ldc != padded_ld(a.n) || (reinterpret_cast<uintptr_t>(a.c) & 3u) != 0) return hipErrorInvalidValue;
  if (a.modulus < 2 || a.modulus > 256) return hipErrorInvalidValue;
  const int64_t groups_per_row = a.ldc / 4;
  const int64_t total = groups_per_row * a.m;
  hipLaunchKernelGGL(export_u8_kernel, dim3(grid_for(total)), dim3(256), 0, stream, a, groups_per_row, total);
  return hipGetLastError();
}

}  // namespace rns8x
