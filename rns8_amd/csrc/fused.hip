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
// slower than two packs and the split-K GEMM (92 against 83 us of kernels).
//
// Work split: a workgroup owns a 128 x 128 output tile, a group of up to four
// planes and one K slice; its four waves each hold a 64 x 64 quadrant of all
// four planes (4 planes x 2 x 2 blocks of v_mfma_i32_32x32x32_i8, 256
// accumulator registers), so one workgroup runs per CU. The raw int64 tiles
// of each 32-deep K step (32 KB of A, 32 KB of B) are loaded straight into
// LDS two steps ahead, holding no registers while in flight. Per step every
// thread reads 16 native elements of A (one row, 16 consecutive k) and 16 of B
// (one column, 16 consecutive k) from LDS, reduces them to centered residues
// for each plane of the group with the pack's arithmetic (two v_dot4_u32_u8
// and a 24-bit quotient, tables.hpp), and stores them into a k-contiguous
// residue stage, so every MFMA fragment is one ds_read_b128. Each element is
// reduced once per plane, as in the packs. LDS: a 32 KB residue stage and two
// 64 KB raw stages, 160 KB.
//
// Each slice reduces its int32 sums to centered int8 residues in the
// epilogue and stores them into its own slot of the workspace; a finalize
// kernel adds the slices' residues and reduces once more. Partial residues
// are a quarter of the bytes of int32 partial sums, and slices of at most
// 65536 K keep every int32 sum exact.
#include <algorithm>
#include <type_traits>

#include "dma.hpp"
#include "int_ops.hpp"
#include "kernels.hpp"

namespace rns8x {
namespace {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef unsigned long long v2u64 __attribute__((ext_vector_type(2)));

constexpr int kTileM = 128;                           // output rows per workgroup
constexpr int kTileN = 128;                           // output columns per workgroup
constexpr int kStepK = 32;                            // K per step (one MFMA depth)
constexpr int kGroupPlanes = 4;                       // planes per workgroup
constexpr int kALds = kTileM * kStepK;                // 4 KB of residues: 128 rows x 32 k
constexpr int kBLds = kTileN * kStepK;                // 4 KB of residues: 128 columns x 32 k
constexpr int kPlaneLds = kALds + kBLds;
constexpr int kResLds = kGroupPlanes * kPlaneLds;     // 32 KB: the residue stage
constexpr int kRawA = kTileM * kStepK * 8;            // 32 KB: 128 rows x 256 bytes of native A
constexpr int kRawB = kStepK * kTileN * 8;            // 32 KB: 32 k rows x 1 KB of native B
constexpr int kRawLds = kRawA + kRawB;
constexpr int kLdsBytes = kResLds + 2 * kRawLds;      // 160 KB: residues + two raw stages
constexpr int kDmaPerWave = (kRawLds / 1024) / 4;     // 16 one-KB loads per wave per step
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
// every slice holds at least one K element, 16-byte aligned operands with
// even row strides, and row strides below 2^21 elements. NP is a template
// parameter so that every accumulator is updated unconditionally and stays
// in its AGPRs.
template <bool Signed, int NP>
__global__ __launch_bounds__(256, 1) void fused_native_kernel(FusedArgs a, PlaneConsts pc, uint32_t tiles_n,
                                                              uint32_t plane_base) {
  __shared__ __attribute__((aligned(16))) int8_t lds[kLdsBytes];
  int8_t* const res = lds;                 // residue stage
  int8_t* const raw0 = lds + kResLds;      // raw stages: A rows then B k rows
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
  const int64_t rows_valid = min(static_cast<int64_t>(kTileM), a.m - m0);

  // Raw loads, straight into LDS (16 bytes per lane, no registers held while
  // in flight). Wave w loads A rows 32w .. 32w+31 as 8 blocks of 4 rows x 256
  // bytes, and B k rows 8w .. 8w+7 as 8 blocks of 1 KB. In A, the 16-byte
  // chunk c of row r is stored at chunk position c ^ (r & 7) of its LDS row,
  // so the conversion's reads (two rows per 8-lane group, same chunk index)
  // fall on distinct banks. Rows past the operand read 0 through the buffer
  // resources' ranges; k past the slice and columns past n are zeroed when
  // converted (within a row they may hold the row padding of a strided
  // operand).
  const uint32_t lds_raw0 = lds_address(raw0);
  uint32_t a_voff[8], b_voff[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int row = 32 * wave + 4 * j + (lane >> 4);
    const int chunk = (lane & 15) ^ (row & 7);
    a_voff[j] = static_cast<uint32_t>(row) * static_cast<uint32_t>(a.lda) * 8u + 16u * static_cast<uint32_t>(chunk);
    const int kr = 8 * wave + j;
    b_voff[j] = static_cast<uint32_t>(kr) * static_cast<uint32_t>(a.ldb) * 8u + 16u * static_cast<uint32_t>(lane);
  }
  const uint64_t* const abase = static_cast<const uint64_t*>(a.a) + m0 * a.lda;
  const uint64_t* const bbase = static_cast<const uint64_t*>(a.b) + n0;
  auto issue = [&](int s, int stage) {
    const int64_t k0 = kb + static_cast<int64_t>(kStepK) * s;
    // The ranges end at the operands' last logical elements (row rows_valid - 1,
    // column k - 1 of A; k row k0 + krows - 1, column n - 1 of B), so no lane
    // reads past an allocation of exactly (m - 1) * lda + k resp.
    // (k - 1) * ldb + n elements; lanes past them read 0.
    const v4i ra = buffer_rsrc(abase + k0, ((rows_valid - 1) * a.lda + a.k - k0) * 8);
    const int64_t krows = min(static_cast<int64_t>(kStepK), a.k - k0);
    const v4i rb = buffer_rsrc(bbase + k0 * a.ldb, ((krows - 1) * a.ldb + a.n - n0) * 8);
    const uint32_t dst = lds_raw0 + static_cast<uint32_t>(stage * kRawLds);
#pragma unroll
    for (int j = 0; j < 8; ++j) dma16(dst + static_cast<uint32_t>((8 * wave + j) * 1024), a_voff[j], ra);
#pragma unroll
    for (int j = 0; j < 8; ++j) dma16(dst + static_cast<uint32_t>(kRawA + (8 * wave + j) * 1024), b_voff[j], rb);
  };

  // Conversion roles: A row a_r, k 16*a_h .. +15; B column b_c, k 16*b_h .. +15.
  const int a_r = t >> 1, a_h = t & 1;
  const int b_c = t & 127, b_h = t >> 7;
  const bool b_ok = n0 + b_c < a.n;
  auto convert = [&](int s, int stage) {
    const int64_t k0 = kb + static_cast<int64_t>(kStepK) * s;
    const int8_t* const raw = raw0 + stage * kRawLds;
    uint32_t alo[16], ahi[16], blo[16], bhi[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int chunk = (8 * a_h + j) ^ (a_r & 7);
      const v4i v = *reinterpret_cast<const v4i*>(raw + a_r * 256 + 16 * chunk);
      const bool ok0 = k0 + 16 * a_h + 2 * j < ke, ok1 = k0 + 16 * a_h + 2 * j + 1 < ke;
      alo[2 * j] = ok0 ? static_cast<uint32_t>(v[0]) : 0u;
      ahi[2 * j] = ok0 ? static_cast<uint32_t>(v[1]) : 0u;
      alo[2 * j + 1] = ok1 ? static_cast<uint32_t>(v[2]) : 0u;
      ahi[2 * j + 1] = ok1 ? static_cast<uint32_t>(v[3]) : 0u;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const v2i v = *reinterpret_cast<const v2i*>(raw + kRawA + (16 * b_h + e) * 1024 + 8 * b_c);
      const bool ok = b_ok && k0 + 16 * b_h + e < ke;
      blo[e] = ok ? static_cast<uint32_t>(v[0]) : 0u;
      bhi[e] = ok ? static_cast<uint32_t>(v[1]) : 0u;
    }
    if (Signed) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        ahi[e] ^= 0x80000000u;
        bhi[e] ^= 0x80000000u;
      }
    }
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) {
      const ModulusConsts mc = pc.mod[p0 + pl];
      const uint32_t off = Signed ? mc.off_i64 : mc.off_u64;
      const v4i wa = {static_cast<int>(residues4(alo, ahi, 0, mc, off)), static_cast<int>(residues4(alo, ahi, 1, mc, off)),
                      static_cast<int>(residues4(alo, ahi, 2, mc, off)), static_cast<int>(residues4(alo, ahi, 3, mc, off))};
      const v4i wb = {static_cast<int>(residues4(blo, bhi, 0, mc, off)), static_cast<int>(residues4(blo, bhi, 1, mc, off)),
                      static_cast<int>(residues4(blo, bhi, 2, mc, off)), static_cast<int>(residues4(blo, bhi, 3, mc, off))};
      *reinterpret_cast<v4i*>(res + pl * kPlaneLds + a_r * kStepK + 16 * a_h) = wa;
      *reinterpret_cast<v4i*>(res + pl * kPlaneLds + kALds + b_c * kStepK + 16 * b_h) = wb;
    }
  };

  // Fragments: lane l takes row (A) or column (B) l & 31 of a 32-block and the
  // 16 k values 16*(l >> 5) .. +15, one ds_read_b128 each. With B as src0 and
  // A as src1, register 4g+e of acc[pl][i][j] holds C[row][col] of plane
  // p0 + pl with row = m0 + 64*wm + 32*i + (l & 31) and col = n0 + 64*wn +
  // 32*j + 8*g + 4*(l >> 5) + e.
  v16i acc[NP][2][2];
#pragma unroll
  for (int pl = 0; pl < NP; ++pl)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[pl][i][j] = v16i{};
  const int frag = (lane & 31) * kStepK + 16 * (lane >> 5);
  auto mma = [&]() {
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) {
      v4i af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const v4i*>(res + pl * kPlaneLds + (64 * wm + 32 * i) * kStepK + frag);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *reinterpret_cast<const v4i*>(res + pl * kPlaneLds + kALds + (64 * wn + 32 * j) * kStepK + frag);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[pl][i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j], af[i], acc[pl][i][j], 0, 0, 0);
    }
  };

  // Pipeline: the raw data of steps s+1 and s+2 are in flight (or landed)
  // while step s is converted and multiplied. Every step issues exactly
  // kDmaPerWave loads per wave (past the last step the last step's data is
  // loaded again into the free stage and never converted, so the vmcnt
  // bookkeeping stays uniform); loads complete in order, so before
  // converting step s each wave waits until only the newest step's loads are
  // outstanding, and the barrier after that wait publishes every wave's loads
  // of step s.
  issue(0, 0);
  issue(min(1, steps - 1), 1);
  for (int s = 0; s < steps; ++s) {
    __builtin_amdgcn_s_waitcnt(wait_vm(kDmaPerWave));  // step s landed (this wave's part)
    __syncthreads();                                  // every wave's part; step s-1's MFMAs retired
    convert(s, s & 1);
    __syncthreads();                                  // residues of step s stored; raw stage s&1 free
    // the raw stage just converted takes step s+2 (a repeat of the last step
    // past the end, never converted)
    issue(min(s + 2, steps - 1), s & 1);
    mma();
  }
  __builtin_amdgcn_s_waitcnt(wait_vm(0));  // no load outlives the workgroup's LDS

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
        for (int j = 0; j < 2; ++j) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int64_t col = n0 + 64 * wn + 32 * j + 8 * g + 4 * (lane >> 5);
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

bool fused_operands_ok(const void* a, int64_t lda, const void* b, int64_t ldb) {
  return (reinterpret_cast<uintptr_t>(a) & 15u) == 0 && (reinterpret_cast<uintptr_t>(b) & 15u) == 0 && lda % 2 == 0 &&
         ldb % 2 == 0 && lda < (int64_t{1} << 21) && ldb < (int64_t{1} << 21);
}

bool choose_fused_shape(int64_t m, int64_t n, int64_t k, uint32_t nplanes, int64_t ldc, FusedShape& out) {
  out = FusedShape{};
  if (m <= 0 || n <= 0 || k <= 0 || nplanes == 0 || nplanes > kMaxPrefix || ldc < n || ldc % 16 != 0) return false;
  if (m >= (int64_t{1} << 31) || n >= (int64_t{1} << 31)) return false;
  const int64_t tiles = ((m + kTileM - 1) / kTileM) * ((n + kTileN - 1) / kTileN);
  const int64_t groups = (nplanes + kGroupPlanes - 1) / kGroupPlanes;
  if (tiles >= (int64_t{1} << 31)) return false;
  // about one workgroup per CU, slices of at least kMinSliceK and at most
  // kMaxSliceK, every slice non-empty
  const int64_t target = (256 + tiles * groups - 1) / (tiles * groups);
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

bool fused_args_ok(const FusedArgs& a) {
  FusedShape expect;
  if (!a.a || !a.b || !a.c || !a.ws || a.lda < a.k || a.ldb < a.n) return false;
  if (!choose_fused_shape(a.m, a.n, a.k, a.nplanes, a.ldc, expect) || expect.slices != a.shape.slices ||
      expect.k_slice != a.shape.k_slice)
    return false;
  if (a.pitch_c < a.m * a.ldc || (reinterpret_cast<uintptr_t>(a.c) & 3u) != 0 ||
      (reinterpret_cast<uintptr_t>(a.ws) & 3u) != 0)
    return false;
  // the direct-to-LDS loads read 16-byte chunks at 32-bit byte offsets
  return fused_operands_ok(a.a, a.lda, a.b, a.ldb);
}

hipError_t launch_fused_native(const FusedArgs& a, const PlaneConsts& consts, hipStream_t stream) {
  if (!fused_args_ok(a)) return hipErrorInvalidValue;
  const uint32_t tiles_n = static_cast<uint32_t>((a.n + kTileN - 1) / kTileN);
  const uint32_t tiles = static_cast<uint32_t>((a.m + kTileM - 1) / kTileM) * tiles_n;
  const bool sgn = a.kind == NativeKind::I64;
  // full groups of four planes in one grid, the remaining 1-3 planes in another
  const uint32_t full = a.nplanes / kGroupPlanes;
  const uint32_t rest = a.nplanes - full * kGroupPlanes;
  auto launch = [&](auto np, uint32_t groups, uint32_t base) {
    constexpr int NP = decltype(np)::value;
    const dim3 grid(tiles, a.shape.slices, groups);
    if (sgn)
      hipLaunchKernelGGL((fused_native_kernel<true, NP>), grid, dim3(256), 0, stream, a, consts, tiles_n, base);
    else
      hipLaunchKernelGGL((fused_native_kernel<false, NP>), grid, dim3(256), 0, stream, a, consts, tiles_n, base);
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
