// Fused native-input plane GEMM: C's residue planes straight from int64 /
// uint64 device operands, the pack folded into the GEMM's operand loads
// (reference hip_direct_gemm_native_kernels.cuh:9-193 converts native
// operands inside its tile loads the same way, one plane per launch slice).
//
// Scope: outputs too small to fill the chip, so the work is split along K
// (tall-skinny products such as 128 x 128 x 65536), where the packed planes
// would be read only once by the GEMM; the fused launch never stores
// residues to HBM. For large outputs every operand panel is read by many
// output tiles and packing once is cheaper, so the host offers the fused path
// only below a workspace limit. Measured at 128 x 128 x 65536 it is still
// slower than two packs and the split-K GEMM (96 against 83 us of kernels):
// it does 1.5 times the packs' residue arithmetic (A's elements are reduced
// once per 64-column tile and per plane group), which keeps its VALU about
// half busy, and its waves wait on their loads for most of the rest.
//
// Work split: a workgroup owns a 128 x 64 output tile, a group of up to four
// planes and one K slice; two workgroups run per CU. Its four waves each hold
// a 64 x 32 part of all four planes (4 planes x 2 blocks of
// v_mfma_i32_32x32x32_i8, 128 accumulator registers). Per 32-deep K step
// every thread loads 16 native elements of A (two consecutive k of eight rows,
// so a wave's load covers whole row segments) and 8 of B (one column, 8
// consecutive k), reduces them to centered residues for each plane of the
// group with the pack's arithmetic (two v_dot4_u32_u8 and a 24-bit quotient,
// tables.hpp), and stores them into a k-contiguous LDS layout, so every MFMA
// fragment is one ds_read_b128. LDS is double-buffered: the next step's loads
// and residues overlap this step's MFMAs.
//
// Each slice reduces its int32 sums to centered int8 residues in the
// epilogue and stores them into its own slot of the workspace; a finalize
// kernel adds the slices' residues and reduces once more. Partial residues
// are a quarter of the bytes of int32 partial sums, and slices of at most
// 65536 K keep every int32 sum exact.
#include <algorithm>
#include <type_traits>

#include "int_ops.hpp"
#include "kernels.hpp"

namespace rns8x {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef unsigned long long v2u64 __attribute__((ext_vector_type(2)));

constexpr int kTileM = 128;                           // output rows per workgroup
constexpr int kTileN = 64;                            // output columns per workgroup
constexpr int kStepK = 32;                            // K per step (one MFMA depth)
constexpr int kGroupPlanes = 4;                       // planes per workgroup
constexpr int kALds = kTileM * kStepK;                // 4 KB: 128 rows x 32 k
constexpr int kBLds = kTileN * kStepK;                // 2 KB: 64 columns x 32 k
constexpr int kPlaneLds = kALds + kBLds;              // A block, then B block
constexpr int kStageLds = kGroupPlanes * kPlaneLds;   // 24 KB
constexpr int64_t kMaxSliceK = 65536;                 // |int32 sum| <= 65536 * 128 * 128 = 2^30
constexpr int64_t kMinSliceK = 512;                   // 16 steps: amortizes the epilogue
constexpr uint64_t kMaxWorkspace = uint64_t{64} << 20;

// Centered residues of native values 4q .. 4q+3 (split in 32-bit halves, the
// sign bit of signed inputs already flipped) for one modulus, packed
// little-endian
// (reference cpu_reference.cpp:53-130; the same arithmetic as the pack kernel).
template <int N>
__device__ __forceinline__ uint32_t residues4(const uint32_t (&lo)[N], const uint32_t (&hi)[N], int q,
                                              const ModulusConsts& mc, uint32_t off) {
  if (mc.m == 256u) return pack_low_bytes(lo[4 * q], lo[4 * q + 1], lo[4 * q + 2], lo[4 * q + 3]);
  const uint32_t m_comp = 256u - mc.m;
  uint32_t r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t t = __builtin_amdgcn_udot4(lo[4 * q + e], mc.pow_lo, off, false);
    r[e] = mod_low_byte(__builtin_amdgcn_udot4(hi[4 * q + e], mc.pow_hi, t, false), mc.pq_shift, mc.pq_recip, m_comp);
  }
  return pack_centered(r[0], r[1], r[2], r[3], mc.half * 0x00010001u);
}

// Grid: x = output tile (tiles_n per tile row), y = K slice, z = plane group
// (planes p0 .. p0 + NP - 1, p0 = plane_base + 4 * z). The host guarantees
// every slice holds at least one K element and (for Vec) 16-byte aligned A
// rows. NP is a template parameter so that every accumulator is updated
// unconditionally and stays in its AGPRs.
template <bool Signed, bool Vec, int NP>
__global__ __launch_bounds__(256, 2) void fused_native_kernel(FusedArgs a, PlaneConsts pc, uint32_t tiles_n,
                                                              uint32_t plane_base) {
  __shared__ __attribute__((aligned(16))) int8_t lds[2 * kStageLds];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const uint32_t tr = blockIdx.x / tiles_n;
  const uint32_t tc = blockIdx.x - tr * tiles_n;
  const int64_t m0 = static_cast<int64_t>(tr) * kTileM;
  const int64_t n0 = static_cast<int64_t>(tc) * kTileN;
  const uint32_t slice = blockIdx.y;
  const uint32_t p0 = plane_base + blockIdx.z * kGroupPlanes;
  const int64_t kb = static_cast<int64_t>(slice) * a.shape.k_slice;
  const int64_t ke = min(kb + a.shape.k_slice, a.k);
  const int steps = static_cast<int>((ke - kb + kStepK - 1) / kStepK);

  // Loader roles. A: sixteen threads per row, two consecutive k each, so a
  // wave's load covers four whole 256-byte row segments; thread t holds rows
  // (t >> 4) + 16j, j = 0..7, at k = 2*(t & 15), +1 (element 2j, 2j+1 of its
  // arrays). B: column b_col, k 8*b_q .. +7.
  const int a_r0 = t >> 4, a_k2 = 2 * (t & 15);
  const int b_col = t & 63, b_q = t >> 6;
  const bool b_ok = n0 + b_col < a.n;
  // Rows past m and columns past n read row / column 0, k past the slice
  // reads its last element, and the values are replaced by 0 afterwards: every
  // load is in bounds and unconditional, so a thread's loads are all in flight
  // together (a load under a condition followed by a select waits for each
  // one in turn).
  const uint64_t* const a_base = static_cast<const uint64_t*>(a.a);
  const uint64_t* const b_src = static_cast<const uint64_t*>(a.b) + (b_ok ? n0 + b_col : 0);

  // raw operand words of one step
  struct Raw {
    uint32_t alo[16], ahi[16], blo[8], bhi[8];
  };
  auto load = [&](Raw& raw, int64_t k0) {
    const int64_t ka = k0 + a_k2;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t row = m0 + a_r0 + 16 * j;
      const bool ok = row < a.m;
      const uint64_t* const rp = a_base + (ok ? row * a.lda : 0);
      uint64_t x0, x1;
      if (Vec && ka + 2 <= ke) {
        const v2u64 v = *reinterpret_cast<const v2u64*>(rp + ka);
        x0 = v[0];
        x1 = v[1];
      } else {
        const uint64_t y0 = rp[min(ka, ke - 1)];
        const uint64_t y1 = rp[min(ka + 1, ke - 1)];
        x0 = ka < ke ? y0 : 0ull;  // out of range packs as 0
        x1 = ka + 1 < ke ? y1 : 0ull;
      }
      x0 = ok ? x0 : 0ull;
      x1 = ok ? x1 : 0ull;
      raw.alo[2 * j] = static_cast<uint32_t>(x0);
      raw.ahi[2 * j] = static_cast<uint32_t>(x0 >> 32);
      raw.alo[2 * j + 1] = static_cast<uint32_t>(x1);
      raw.ahi[2 * j + 1] = static_cast<uint32_t>(x1 >> 32);
    }
    const int64_t kk = k0 + 8 * b_q;
    uint64_t y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = b_src[min(kk + e, ke - 1) * a.ldb];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint64_t v = b_ok && kk + e < ke ? y[e] : 0ull;
      raw.blo[e] = static_cast<uint32_t>(v);
      raw.bhi[e] = static_cast<uint32_t>(v >> 32);
    }
    if (Signed) {
#pragma unroll
      for (int e = 0; e < 16; ++e) raw.ahi[e] ^= 0x80000000u;
#pragma unroll
      for (int e = 0; e < 8; ++e) raw.bhi[e] ^= 0x80000000u;
    }
  };
  // residues of the loaded elements for every plane of the group, into stage
  // `stage`: A row r, k at r*32 + k; B column c, k at 4096 + c*32 + k
  auto convert_store = [&](const Raw& raw, int stage) {
    int8_t* const st = lds + stage * kStageLds;
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) {
      {
        const ModulusConsts mc = pc.mod[p0 + pl];
        const uint32_t off = Signed ? mc.off_i64 : mc.off_u64;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          // residues of rows a_r0 + 16*(2q) and + 16*(2q + 1): bytes 0-1 and 2-3
          const uint32_t w = residues4(raw.alo, raw.ahi, q, mc, off);
          *reinterpret_cast<uint16_t*>(st + pl * kPlaneLds + (a_r0 + 32 * q) * kStepK + a_k2) =
              static_cast<uint16_t>(w);
          *reinterpret_cast<uint16_t*>(st + pl * kPlaneLds + (a_r0 + 32 * q + 16) * kStepK + a_k2) =
              static_cast<uint16_t>(w >> 16);
        }
        const v2i wb = {static_cast<int>(residues4(raw.blo, raw.bhi, 0, mc, off)),
                        static_cast<int>(residues4(raw.blo, raw.bhi, 1, mc, off))};
        *reinterpret_cast<v2i*>(st + pl * kPlaneLds + kALds + b_col * kStepK + 8 * b_q) = wb;
      }
    }
  };

  // Fragments: lane l takes row (A) or column (B) l & 31 of a 32-block and the
  // 16 k values 16*(l >> 5) .. +15, one ds_read_b128 each. With B as src0 and
  // A as src1, register 4g+e of acc[pl][i][j] holds C[row][col] of plane
  // p0 + pl with row = m0 + 64*wm + 32*i + (l & 31) and col = n0 + 64*wn +
  // 32*j + 8*g + 4*(l >> 5) + e.
  v16i acc[NP][2][1];
#pragma unroll
  for (int pl = 0; pl < NP; ++pl)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 1; ++j) acc[pl][i][j] = v16i{};
  const int frag = (lane & 31) * kStepK + 16 * (lane >> 5);
  auto mma = [&](int stage) {
    const int8_t* const st = lds + stage * kStageLds;
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) {
      {
        v4i af[2], bf[1];
#pragma unroll
        for (int i = 0; i < 2; ++i)
          af[i] = *reinterpret_cast<const v4i*>(st + pl * kPlaneLds + (64 * wm + 32 * i) * kStepK + frag);
#pragma unroll
        for (int j = 0; j < 1; ++j)
          bf[j] = *reinterpret_cast<const v4i*>(st + pl * kPlaneLds + kALds + (32 * wn + 32 * j) * kStepK + frag);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 1; ++j)
            acc[pl][i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j], af[i], acc[pl][i][j], 0, 0, 0);
      }
    }
  };

  // Step s computes from stage s & 1 while the next step's loads are in
  // flight and its residues go into the other stage, which the barrier ending
  // step s-1 retired.
  Raw raw;
  load(raw, kb);
  convert_store(raw, 0);
  __syncthreads();
  for (int s = 0; s < steps; ++s) {
    const bool more = s + 1 < steps;
    if (more) load(raw, kb + static_cast<int64_t>(kStepK) * (s + 1));
    mma(s & 1);
    if (more) convert_store(raw, (s + 1) & 1);
    __syncthreads();
  }

  // Epilogue: each int32 sum x (|x| <= 2^30) reduced to its centered residue,
  // four columns per dword, into slot [slice][plane][row][col] of the
  // workspace (row stride ldc). Columns in [n, ldc) hold residues of zero
  // sums; rows past m are not stored.
#pragma unroll
  for (int pl = 0; pl < NP; ++pl) {
    {
      const uint32_t plane = p0 + pl;
      const ModulusConsts mc = pc.mod[plane];
      const uint32_t m_comp = 256u - mc.m;
      const uint32_t half2 = mc.half * 0x00010001u;
      int8_t* const w = a.ws + (static_cast<int64_t>(slice) * a.nplanes + plane) * a.m * a.ldc;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int64_t row = m0 + 64 * wm + 32 * i + (lane & 31);
#pragma unroll
        for (int j = 0; j < 1; ++j) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int64_t col = n0 + 32 * wn + 32 * j + 8 * g + 4 * (lane >> 5);
            const Acc4 a4 = acc_read4(acc[pl][i][j], g);
            uint32_t r[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t u = a4.v[e] ^ 0x80000000u;
              r[e] = mc.m == 256u ? u : residue_plus_half(u, mc, m_comp);
            }
            const uint32_t packed = mc.m == 256u ? pack_low_bytes(r[0], r[1], r[2], r[3])
                                                 : pack_centered(r[0], r[1], r[2], r[3], half2);
            if (row < a.m && col < a.ldc) *reinterpret_cast<uint32_t*>(w + row * a.ldc + col) = packed;
          }
        }
      }
    }
  }
}

// Adds the slices' centered residues of four consecutive cells (one dword per
// slice) and writes their centered residue into C (reference
// cpu_reference.cpp:156-311: the plane result is the sum's residue). A block
// covers 32 dwords; its eight 32-thread groups each add every eighth slice,
// so the loads of many slices are in flight at once, and group 0 combines
// the eight partial sums.
constexpr int kFinalWords = 32;
constexpr int kFinalGroups = 8;
__global__ __launch_bounds__(256) void residue_finalize_kernel(const int8_t* ws, int8_t* c, int64_t m, int64_t ldc,
                                                               int64_t pitch_c, uint32_t nplanes, uint32_t slices,
                                                               PlaneConsts pc) {
  __shared__ int32_t part[kFinalGroups][kFinalWords][4];
  const int64_t words_per_plane = m * ldc / 4;
  const int64_t total = words_per_plane * nplanes;
  const int64_t slice_words = static_cast<int64_t>(nplanes) * words_per_plane;
  const uint32_t* const src = reinterpret_cast<const uint32_t*>(ws);
  const int lw = threadIdx.x % kFinalWords;
  const int grp = threadIdx.x / kFinalWords;
  for (int64_t w0 = static_cast<int64_t>(blockIdx.x) * kFinalWords; w0 < total;
       w0 += static_cast<int64_t>(gridDim.x) * kFinalWords) {
    const int64_t w = w0 + lw;
    int32_t sum[4] = {0, 0, 0, 0};
    if (w < total) {
      for (uint32_t s = grp; s < slices; s += kFinalGroups) {
        const uint32_t v = src[static_cast<int64_t>(s) * slice_words + w];
#pragma unroll
        for (int e = 0; e < 4; ++e) sum[e] += static_cast<int32_t>(static_cast<int8_t>(v >> (8 * e)));
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) part[grp][lw][e] = sum[e];
    __syncthreads();
    if (grp == 0 && w < total) {
#pragma unroll
      for (int g = 1; g < kFinalGroups; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) sum[e] += part[g][lw][e];
      const uint32_t plane = static_cast<uint32_t>(w / words_per_plane);
      const int64_t in_plane = w - static_cast<int64_t>(plane) * words_per_plane;
      const ModulusConsts mc = pc.mod[plane];
      uint32_t r[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = residue_plus_half(static_cast<uint32_t>(sum[e]) ^ 0x80000000u, mc, 256u - mc.m);
      *reinterpret_cast<uint32_t*>(c + static_cast<int64_t>(plane) * pitch_c + in_plane * 4) =
          pack_centered(r[0], r[1], r[2], r[3], mc.half * 0x00010001u);
    }
    __syncthreads();
  }
}

}  // namespace

bool choose_fused_shape(int64_t m, int64_t n, int64_t k, uint32_t nplanes, int64_t ldc, FusedShape& out) {
  out = FusedShape{};
  if (m <= 0 || n <= 0 || k <= 0 || nplanes == 0 || nplanes > kMaxPrefix || ldc < n || ldc % 16 != 0) return false;
  if (m >= (int64_t{1} << 31) || n >= (int64_t{1} << 31)) return false;
  const int64_t tiles = ((m + kTileM - 1) / kTileM) * ((n + kTileN - 1) / kTileN);
  const int64_t groups = (nplanes + kGroupPlanes - 1) / kGroupPlanes;
  if (tiles >= (int64_t{1} << 31)) return false;
  // about one workgroup per CU, slices of at least kMinSliceK and at most
  // kMaxSliceK, every slice non-empty
  const int64_t target = (512 + tiles * groups - 1) / (tiles * groups);
  int64_t slices = std::max((k + kMaxSliceK - 1) / kMaxSliceK, std::min(target, (k + kMinSliceK - 1) / kMinSliceK));
  slices = std::max<int64_t>(slices, 1);
  int64_t k_slice = (k + slices - 1) / slices;
  k_slice = (k_slice + kStepK - 1) / kStepK * kStepK;
  slices = (k + k_slice - 1) / k_slice;
  if (slices > 65535) return false;
  const uint64_t bytes = static_cast<uint64_t>(slices) * nplanes * static_cast<uint64_t>(m) * static_cast<uint64_t>(ldc);
  if (bytes > kMaxWorkspace) return false;
  out.slices = static_cast<uint32_t>(slices);
  out.k_slice = k_slice;
  out.ws_bytes = bytes;
  return true;
}

hipError_t launch_fused_native(const FusedArgs& a, const PlaneConsts& consts, hipStream_t stream) {
  FusedShape expect;
  if (!a.a || !a.b || !a.c || !a.ws || a.lda < a.k || a.ldb < a.n) return hipErrorInvalidValue;
  if (!choose_fused_shape(a.m, a.n, a.k, a.nplanes, a.ldc, expect) || expect.slices != a.shape.slices ||
      expect.k_slice != a.shape.k_slice)
    return hipErrorInvalidValue;
  if (a.pitch_c < a.m * a.ldc || (reinterpret_cast<uintptr_t>(a.c) & 3u) != 0 ||
      (reinterpret_cast<uintptr_t>(a.ws) & 3u) != 0)
    return hipErrorInvalidValue;
  const uint32_t tiles_n = static_cast<uint32_t>((a.n + kTileN - 1) / kTileN);
  const uint32_t tiles = static_cast<uint32_t>((a.m + kTileM - 1) / kTileM) * tiles_n;
  const bool vec = (reinterpret_cast<uintptr_t>(a.a) & 15u) == 0 && (a.lda % 2) == 0;
  const bool sgn = a.kind == NativeKind::I64;
  // full groups of four planes in one grid, the remaining 1-3 planes in another
  const uint32_t full = a.nplanes / kGroupPlanes;
  const uint32_t rest = a.nplanes - full * kGroupPlanes;
  auto launch = [&](auto np, uint32_t groups, uint32_t base) {
    constexpr int NP = decltype(np)::value;
    const dim3 grid(tiles, a.shape.slices, groups);
    if (sgn && vec)
      hipLaunchKernelGGL((fused_native_kernel<true, true, NP>), grid, dim3(256), 0, stream, a, consts, tiles_n, base);
    else if (sgn)
      hipLaunchKernelGGL((fused_native_kernel<true, false, NP>), grid, dim3(256), 0, stream, a, consts, tiles_n, base);
    else if (vec)
      hipLaunchKernelGGL((fused_native_kernel<false, true, NP>), grid, dim3(256), 0, stream, a, consts, tiles_n, base);
    else
      hipLaunchKernelGGL((fused_native_kernel<false, false, NP>), grid, dim3(256), 0, stream, a, consts, tiles_n, base);
  };
  if (full) launch(std::integral_constant<int, kGroupPlanes>{}, full, 0);
  const uint32_t base = full * kGroupPlanes;
  if (rest == 1) launch(std::integral_constant<int, 1>{}, 1, base);
  if (rest == 2) launch(std::integral_constant<int, 2>{}, 1, base);
  if (rest == 3) launch(std::integral_constant<int, 3>{}, 1, base);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t words = static_cast<int64_t>(a.nplanes) * a.m * a.ldc / 4;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((words + kFinalWords - 1) / kFinalWords, 4096));
  hipLaunchKernelGGL(residue_finalize_kernel, dim3(blocks), dim3(256), 0, stream, a.ws, a.c, a.m, a.ldc, a.pitch_c,
                     a.nplanes, a.shape.slices, consts);
  return hipGetLastError();
}

}  // namespace rns8x
