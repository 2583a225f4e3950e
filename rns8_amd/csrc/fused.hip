// Fused native-input plane GEMM: C's residue planes straight from int64 /
// uint64 device operands, the pack folded into the GEMM's operand loads
// (reference hip_direct_gemm_native_kernels.cuh:9-193 converts native
// operands inside its tile loads the same way, one plane per launch slice).
//
// Scope: outputs too small to fill the chip, so the work is split along K
// (tall-skinny products such as 128 x 128 x 65536). Each native element is
// read from HBM once and reduced once per plane; no residue plane of A or B is
// ever stored. For large outputs every operand panel would be read by many
// output tiles and packing once is cheaper, so the host offers the fused path
// only below a workspace limit.
//
// Work split: a workgroup owns a 128 x 128 output tile, a pair of planes and
// one K slice. Its twelve waves run three per SIMD: two converter waves and
// one MFMA wave each (a single wave issues a VALU instruction only every six
// or seven cycles, so the conversion needs two waves per SIMD to keep the VALU
// busy, and the MFMAs issue from a third). Roles:
//   * conversion: waves 0-3 take A, waves 4-7 take B, and every load is
//     coalesced: an A load covers four rows x 32 k (16 lanes per 256-byte row
//     segment, two k per lane), a B load one k row x 128 columns (two columns
//     per lane). A lane thus holds two k of eight rows (A) or eight k of two
//     columns (B). Both roles issue eight 16-byte loads per step; the raw
//     values of step s+2 are requested while step s is converted. Each lane
//     reduces its 16 elements for both planes (the pack's arithmetic: two
//     v_dot4_u32_u8 and a 24-bit quotient, or one dot product when every
//     element of the wave's step fits in 32 bits) and stores its residues
//     into the k-contiguous stage (2 bytes per A row, 8 per B column);
//   * MFMA: wave 8 + q multiplies both planes of the pair over the 64 x 64
//     quadrant q (2 x 2 blocks of v_mfma_i32_32x32x32_i8 per plane, 128
//     accumulator registers), one step behind the conversion: the residue
//     stages are double-buffered and one barrier per step separates a stage's
//     writers from its readers.
// Residue stage layout per plane and operand: [2 k-chunks][128 rows or
// columns][16 bytes], so both the conversion's stores and the fragment reads
// (lane l: row or column l & 31 of a block, k-chunk l >> 5) are contiguous
// 512-byte runs, free of bank conflicts. LDS: 2 stages x 2 planes x 8 KB.
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

constexpr int kThreads = 1024;                       // sixteen waves, four per SIMD
constexpr int kTileM = 128;                          // output rows per workgroup
constexpr int kTileN = 128;                          // output columns per workgroup
constexpr int kStepK = 32;                           // K per step (one MFMA depth)
constexpr int kGroupPlanes = 2;                      // planes per workgroup
constexpr int kChunkLds = 128 * 16;                  // one k-chunk of 128 rows or columns
constexpr int kOperandLds = 2 * kChunkLds;           // 4 KB: 128 x 32 residues
constexpr int kPlaneLds = 2 * kOperandLds;           // A then B
constexpr int kStageLds = kGroupPlanes * kPlaneLds;  // 16 KB
constexpr int kLdsBytes = 2 * kStageLds;             // two stages
constexpr int64_t kMaxSliceK = 65536;                // |int32 sum| <= 65536 * 128 * 128 = 2^30
constexpr int64_t kMinSliceK = 512;                  // 16 steps: amortizes the epilogue
constexpr uint64_t kMaxWorkspace = uint64_t{64} << 20;
constexpr uint32_t kOutOfRange = 0x80000000u;        // a buffer offset past every resource

// A lane's four 16-byte loads of one step, as issued. Element (j, h) is
// v[j][2h] (low half) and v[j][2h + 1] (high half): for an A lane row 4j +
// (lane >> 4) of its wave's 16 rows at k = 2 (lane & 15) + h, for a B lane k =
// j of its wave's 4 k rows at column h of its column pair.
struct Raw {
  v4i v[4];
};

// Grid: x = output tile (tiles_n per tile row), y = K slice, z = plane pair
// (planes p0 .. p0 + NP - 1, p0 = plane_base + 2 * z). The host guarantees
// every slice holds at least one K element, 16-byte aligned operands with
// even row strides, and row strides below 2^21 elements.
template <bool Signed, int NP>
__global__ __launch_bounds__(kThreads, 1) void fused_native_kernel(FusedArgs a, PlaneConsts pc, uint32_t tiles_n,
                                                                   uint32_t plane_base) {
  __shared__ __attribute__((aligned(16))) int8_t lds[kLdsBytes];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const uint32_t tr = blockIdx.x / tiles_n;
  const uint32_t tc = blockIdx.x - tr * tiles_n;
  const int64_t m0 = static_cast<int64_t>(tr) * kTileM;
  const int64_t n0 = static_cast<int64_t>(tc) * kTileN;
  const uint32_t slice = blockIdx.y;
  const uint32_t p0 = plane_base + blockIdx.z * kGroupPlanes;
  const int64_t kb = static_cast<int64_t>(slice) * a.shape.k_slice;
  const int64_t ke = min(kb + a.shape.k_slice, a.k);
  const int steps = static_cast<int>((ke - kb + kStepK - 1) / kStepK);
  const bool ragged = (ke - kb) % kStepK != 0;  // the last step ends inside its 32 k
  const int64_t rows_valid = min(static_cast<int64_t>(kTileM), a.m - m0);

  // ---- conversion ------------------------------------------------------------
  // Waves 0-7 take A, waves 8-15 take B, and every load is coalesced. A wave
  // c: rows 16c + 4j + (lane >> 4), j = 0..3, at k 2 (lane & 15) and 2 (lane &
  // 15) + 1 of the step (16 lanes per 256-byte row segment, four rows per
  // load). B wave 8 + c: k rows 4c .. 4c + 3 at columns 2 lane and 2 lane + 1
  // (one contiguous 1 KB k row per load). Rows past m and k past the operand
  // read 0 through the resources' ranges, which end at the operands' last
  // logical elements (a row's offset past the last valid row exceeds the
  // range since lda >= k). Column pairs past n get an offset outside every
  // resource. A pair that straddles n reads its second column from the row
  // padding (strides are even); the epilogue stores zero for that column.
  const bool is_a = wave < 8;
  const int c = wave & 7;
  const ModulusConsts mc0 = pc.mod[p0];
  const ModulusConsts mc1 = pc.mod[NP > 1 ? p0 + 1 : p0];
  const int ra = 16 * c + (lane >> 4);                 // an A lane's first row (then +4 per load)
  const int kfirst = is_a ? 2 * (lane & 15) : 4 * c;  // the lane's first k within a step
  const uint32_t lda8 = static_cast<uint32_t>(a.lda) * 8u, ldb8 = static_cast<uint32_t>(a.ldb) * 8u;
  const uint32_t voff = is_a ? static_cast<uint32_t>(ra) * lda8 + 8u * kfirst
                             : (n0 + 2 * lane < a.n ? static_cast<uint32_t>(kfirst) * ldb8 + 16u * lane : kOutOfRange);
  const uint32_t vstride = is_a ? 4u * lda8 : ldb8;  // bytes between a lane's loads
  const uint64_t* const abase = static_cast<const uint64_t*>(a.a) + m0 * a.lda;
  const uint64_t* const bbase = static_cast<const uint64_t*>(a.b) + n0;
  auto load = [&](Raw& x, int s) {
    const int64_t k0 = kb + static_cast<int64_t>(kStepK) * s;
    const int64_t krows = min(static_cast<int64_t>(kStepK), a.k - k0);
    const __amdgpu_buffer_rsrc_t rs =
        is_a ? make_rsrc(abase + k0, ((rows_valid - 1) * a.lda + a.k - k0) * 8)
             : make_rsrc(bbase + k0 * a.ldb, ((krows - 1) * a.ldb + a.n - n0) * 8);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      x.v[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, voff + vstride * j, 0, 0));
  };
  // Elements at k >= ke of the slice's last, ragged step belong to the next
  // slice (or to a row's padding) and count as zero.
  auto mask_tail = [&](Raw& x, int s) {
    const int64_t first = kb + static_cast<int64_t>(kStepK) * s + kfirst;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        if (first + (is_a ? h : j) >= ke) x.v[j][2 * h] = x.v[j][2 * h + 1] = 0;
  };
  // Stage addresses: A rows ra + 4j, k-chunk kfirst / 16, bytes kfirst % 16
  // .. +1 of each row's chunk (one 2-byte store per row); B columns 2 lane and
  // 2 lane + 1, k-chunk kfirst / 16, bytes kfirst % 16 .. +3 of each column's
  // chunk (one 4-byte store per column).
  int8_t* const dst0 = is_a ? lds + (kfirst >> 4) * kChunkLds + ra * 16 + (kfirst & 15)
                            : lds + kOperandLds + (kfirst >> 4) * kChunkLds + 2 * lane * 16 + (kfirst & 15);
  // One plane's 8 residues of the lane, stored into the stage. The reduction
  // runs in phases over the 8 elements (dot products, then shifts, quotients
  // and remainders) so independent chains interleave; the modulus-256 plane
  // (the low byte of each element) is a separate instantiation so that
  // neither form carries the other's selects.
  auto part = [&](auto fast, auto m256c, auto is_a_c, const Raw& x, const ModulusConsts& mc, int8_t* dst) {
    constexpr bool kFast = decltype(fast)::value;
    constexpr bool kM256 = decltype(m256c)::value;
    constexpr bool kA = decltype(is_a_c)::value;
    // r[j][h]: the element's centered residue in its low byte
    uint32_t r[4][2];
    const uint32_t m_comp = 256u - mc.m;
    if constexpr (kM256) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) r[j][h] = static_cast<uint32_t>(x.v[j][2 * h]);
    } else {
      // the fast signed form is the accumulator reduction of lo ^ 2^31
      constexpr bool kI32 = kFast && Signed;
      const uint32_t shift = kI32 ? mc.q_shift : mc.pq_shift;
      const uint32_t recip = kI32 ? mc.q_recip : mc.pq_recip;
      // the offsets less H (each offset is at least H): s - H comes out of
      // the dot products (centered_byte)
      const uint32_t off = (kI32 ? mc.off_i32 : Signed ? mc.off_i64 : mc.off_u64) - mc.half;
      const uint32_t h_sh = in_vgpr(mc.half << shift);
      uint32_t s[4][2], q[4][2];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t lo = static_cast<uint32_t>(x.v[j][2 * h]);
          s[j][h] = __builtin_amdgcn_udot4(kI32 ? lo ^ 0x80000000u : lo, mc.pow_lo, off, false);
        }
      if constexpr (!kFast) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t hi = static_cast<uint32_t>(x.v[j][2 * h + 1]);
            s[j][h] = __builtin_amdgcn_udot4(Signed ? hi ^ 0x80000000u : hi, mc.pow_hi, s[j][h], false);
          }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) q[j][h] = (s[j][h] << shift) + h_sh;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) q[j][h] = mulhi_u24(q[j][h], recip);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) r[j][h] = mad_u24(q[j][h], m_comp, s[j][h]);
    }
    auto pack4 = [&](uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3) { return pack_low_bytes(r0, r1, r2, r3); };
    if constexpr (kA) {
      // rows 8q and 8q + 4 share a packed dword: its low half goes to one
      // row, its high half to the other
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t w = pack4(r[2 * q][0], r[2 * q][1], r[2 * q + 1][0], r[2 * q + 1][1]);
        *reinterpret_cast<uint16_t*>(dst + 8 * q * 16) = static_cast<uint16_t>(w);
        *reinterpret_cast<uint16_t*>(dst + (8 * q + 4) * 16) = static_cast<uint16_t>(w >> 16);
      }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h)
        *reinterpret_cast<uint32_t*>(dst + 16 * h) = pack4(r[0][h], r[1][h], r[2][h], r[3][h]);
    }
  };
  auto plane_of = [&](auto fast, const Raw& x, const ModulusConsts& mc, int off) {
    if (is_a) {
      if (mc.m == 256u)
        part(fast, std::true_type{}, std::true_type{}, x, mc, dst0 + off);
      else
        part(fast, std::false_type{}, std::true_type{}, x, mc, dst0 + off);
    } else {
      if (mc.m == 256u)
        part(fast, std::true_type{}, std::false_type{}, x, mc, dst0 + off);
      else
        part(fast, std::false_type{}, std::false_type{}, x, mc, dst0 + off);
    }
  };
  auto convert = [&](const Raw& x, int stage) {
    uint32_t wide = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t lo = static_cast<uint32_t>(x.v[j][2 * h]), hi = static_cast<uint32_t>(x.v[j][2 * h + 1]);
        wide |= Signed ? hi ^ static_cast<uint32_t>(static_cast<int32_t>(lo) >> 31) : hi;
      }
    const int off = stage * kStageLds;
    // one branch per wave: the 32-bit form when no lane has a wide element
    if (__builtin_amdgcn_ballot_w64(wide != 0u) == 0u) {
      plane_of(std::true_type{}, x, mc0, off);
      if constexpr (NP > 1) plane_of(std::true_type{}, x, mc1, off + kPlaneLds);
    } else {
      plane_of(std::false_type{}, x, mc0, off);
      if constexpr (NP > 1) plane_of(std::false_type{}, x, mc1, off + kPlaneLds);
    }
  };

  // ---- MFMA ------------------------------------------------------------------
  // Wave w multiplies plane w >> 3 of the pair over rows 64 wm .. 64 wm + 63
  // and columns 64 wn + 32 hn .. + 31 (wm = (w >> 2) & 1, wn = (w >> 1) & 1,
  // hn = w & 1): two v_mfma_i32_32x32x32_i8 per step, 32 accumulator
  // registers. With B as src0 and A as src1, register 4g+e of acc[i] holds
  // C[row][col] with row = m0 + 64 wm + 32 i + (l & 31) and col = n0 + 64 wn +
  // 32 hn + 8 g + 4 (l >> 5) + e.
  const int pl = wave >> 3, wm = (wave >> 2) & 1, wn = (wave >> 1) & 1, hn = wave & 1;
  const bool mfma_wave = pl < NP;
  const int frag = (lane >> 5) * kChunkLds + (lane & 31) * 16;
  v16i acc[2] = {v16i{}, v16i{}};
  auto mma = [&](int stage) {
    if (!mfma_wave) return;
    const int8_t* const sa = lds + stage * kStageLds + pl * kPlaneLds + frag;
    const int8_t* const sb = sa + kOperandLds;
    const v4i bf = *reinterpret_cast<const v4i*>(sb + (64 * wn + 32 * hn) * 16);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const v4i af = *reinterpret_cast<const v4i*>(sa + (64 * wm + 32 * i) * 16);
      acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf, af, acc[i], 0, 0, 0);
    }
  };

  // ---- pipeline ----------------------------------------------------------------
  // Step s: the raw values of step s+1 are requested (unconditionally, so
  // every step has the same loads in flight; past the end the last step is
  // loaded again and never converted), step s-1 (stage (s-1) & 1, converted
  // in the last step) is multiplied and step s is converted into stage s & 1;
  // the barrier that ends the step publishes stage s & 1 and retires every
  // read of stage (s-1) & 1, which step s+1 overwrites. Two register sets
  // hold the raw values (the loop is unrolled by two so each set keeps its
  // registers).
  auto step = [&](Raw& cur, Raw& next, int s) {
    load(next, min(s + 1, steps - 1));
    if (s > 0) mma((s - 1) & 1);
    if (ragged && s == steps - 1) mask_tail(cur, s);
    convert(cur, s & 1);
    __syncthreads();
  };
  Raw r0, r1;
  load(r0, 0);
  for (int s = 0;;) {
    step(r0, r1, s);
    if (++s >= steps) break;
    step(r1, r0, s);
    if (++s >= steps) break;
  }
  mma((steps - 1) & 1);

  // ---- epilogue --------------------------------------------------------------
  // Each int32 sum x (|x| <= 2^30) reduced to its centered residue, four
  // columns per dword, into slot [slice][plane][row][col] of the workspace
  // (row stride ldc). Columns in [n, ldc) are stored as zero; rows past m are
  // not stored.
  if (!mfma_wave) return;
  const uint32_t plane = p0 + pl;
  const ModulusConsts mc = pl == 0 ? mc0 : mc1;
  const CenteredI32 kc = centered_i32_consts(mc);
  int8_t* const w = a.ws + (static_cast<int64_t>(slice) * a.nplanes + plane) * a.m * a.ldc;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t row = m0 + 64 * wm + 32 * i + (lane & 31);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t col = n0 + 64 * wn + 32 * hn + 8 * g + 4 * (lane >> 5);
      uint32_t r[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t u = static_cast<uint32_t>(acc[i][4 * g + e]) ^ 0x80000000u;
        r[e] = mc.m == 256u ? u : centered_residue_i32(u, mc, kc);
      }
      uint32_t packed = pack_low_bytes(r[0], r[1], r[2], r[3]);
      if (col + 4 > a.n) packed &= col >= a.n ? 0u : 0xFFFFFFFFu >> (8 * (col + 4 - a.n));
      if (row < a.m && col < a.ldc) *reinterpret_cast<uint32_t*>(w + row * a.ldc + col) = packed;
    }
  }
}

// Adds the slices' centered residues of 16 consecutive cells (one 16-byte
// chunk per slice) and writes their centered residue into C (reference
// cpu_reference.cpp:156-311: the plane result is the sum's residue). A block
// covers 256 / G chunks; its G thread groups each add every G-th slice, with
// up to four loads in flight per thread, and group 0 combines the G partial
// sums. m * ldc is a multiple of 16 (ldc is).
template <int G>
__global__ __launch_bounds__(256) void residue_finalize_kernel(const int8_t* ws, int8_t* c, int64_t m, int64_t ldc,
                                                               int64_t pitch_c, uint32_t nplanes, uint32_t slices,
                                                               PlaneConsts pc) {
  constexpr int kChunks = 256 / G;
  __shared__ int32_t part[G][16][kChunks];
  const int64_t chunks_per_plane = m * ldc / 16;
  const int64_t total = chunks_per_plane * nplanes;
  const int64_t slice_chunks = static_cast<int64_t>(nplanes) * chunks_per_plane;
  const v4i* const src = reinterpret_cast<const v4i*>(ws);
  const int lc = threadIdx.x % kChunks;
  const int grp = threadIdx.x / kChunks;
  for (int64_t c0 = static_cast<int64_t>(blockIdx.x) * kChunks; c0 < total;
       c0 += static_cast<int64_t>(gridDim.x) * kChunks) {
    const int64_t ch = c0 + lc;
    int32_t sum[16] = {};
    if (ch < total) {
#pragma unroll 4
      for (uint32_t s = grp; s < slices; s += G) {
        const v4i v = src[static_cast<int64_t>(s) * slice_chunks + ch];
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            sum[4 * d + e] += static_cast<int32_t>(static_cast<int8_t>(static_cast<uint32_t>(v[d]) >> (8 * e)));
      }
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) part[grp][e][lc] = sum[e];
    __syncthreads();
    if (grp == 0 && ch < total) {
#pragma unroll
      for (int g = 1; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 16; ++e) sum[e] += part[g][e][lc];
      const uint32_t plane = static_cast<uint32_t>(ch / chunks_per_plane);
      const int64_t in_plane = ch - static_cast<int64_t>(plane) * chunks_per_plane;
      const ModulusConsts mc = pc.mod[plane];
      const CenteredI32 kc = centered_i32_consts(mc);
      v4i out;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        uint32_t r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          r[e] = centered_residue_i32(static_cast<uint32_t>(sum[4 * d + e]) ^ 0x80000000u, mc, kc);
        out[d] = static_cast<int>(pack_low_bytes(r[0], r[1], r[2], r[3]));
      }
      *reinterpret_cast<v4i*>(c + static_cast<int64_t>(plane) * pitch_c + in_plane * 16) = out;
    }
    __syncthreads();
  }
}

}  // namespace

bool fused_operands_ok(const void* a, int64_t lda, const void* b, int64_t ldb, bool skinny) {
  const bool a_ok = (reinterpret_cast<uintptr_t>(a) & 15u) == 0 && lda % 2 == 0 && lda < (int64_t{1} << 21);
  if (skinny) return a_ok && (reinterpret_cast<uintptr_t>(b) & 7u) == 0;
  return a_ok && (reinterpret_cast<uintptr_t>(b) & 15u) == 0 && ldb % 2 == 0 && ldb < (int64_t{1} << 21);
}

bool choose_fused_shape(int64_t m, int64_t n, int64_t k, uint32_t nplanes, int64_t ldc, FusedShape& out) {
  out = FusedShape{};
  if (m <= 0 || n <= 0 || k <= 0 || nplanes == 0 || nplanes > kMaxPrefix || ldc < n || ldc % 16 != 0) return false;
  // results at most 16 columns wide: the skinny form (fused_skinny.hip)
  if (n <= 16 && ldc == 16 && fused_skinny_shape(m, n, k, nplanes, out)) return true;
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
      expect.k_slice != a.shape.k_slice || expect.skinny != a.shape.skinny || expect.ws_bytes != a.shape.ws_bytes)
    return false;
  // the finalize moves 16-byte chunks of the workspace and of C's planes
  if (a.pitch_c < a.m * a.ldc || a.pitch_c % 16 != 0 || (reinterpret_cast<uintptr_t>(a.c) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(a.ws) & 15u) != 0)
    return false;
  // the operand loads read 16-byte chunks at 32-bit byte offsets
  return fused_operands_ok(a.a, a.lda, a.b, a.ldb, a.shape.skinny != 0);
}

hipError_t launch_fused_native(const FusedArgs& a, const PlaneConsts& consts, hipStream_t stream) {
  if (!fused_args_ok(a)) return hipErrorInvalidValue;
  if (a.shape.skinny) return launch_fused_skinny(a, consts, stream);
  const uint32_t tiles_n = static_cast<uint32_t>((a.n + kTileN - 1) / kTileN);
  const uint32_t tiles = static_cast<uint32_t>((a.m + kTileM - 1) / kTileM) * tiles_n;
  const bool sgn = a.kind == NativeKind::I64;
  // full pairs of planes in one grid, an odd last plane in another
  const uint32_t full = a.nplanes / kGroupPlanes;
  const uint32_t rest = a.nplanes - full * kGroupPlanes;
  auto launch = [&](auto np, uint32_t groups, uint32_t base) {
    constexpr int NP = decltype(np)::value;
    const dim3 grid(tiles, a.shape.slices, groups);
    if (sgn)
      hipLaunchKernelGGL((fused_native_kernel<true, NP>), grid, dim3(kThreads), 0, stream, a, consts, tiles_n, base);
    else
      hipLaunchKernelGGL((fused_native_kernel<false, NP>), grid, dim3(kThreads), 0, stream, a, consts, tiles_n, base);
  };
  if (full) launch(std::integral_constant<int, kGroupPlanes>{}, full, 0);
  if (rest) launch(std::integral_constant<int, 1>{}, 1, full * kGroupPlanes);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_residue_finalize(a.ws, a.c, a.m, a.ldc, a.pitch_c, a.nplanes, a.shape.slices, consts, stream);
}

hipError_t launch_residue_finalize(const int8_t* ws, int8_t* c, int64_t m, int64_t ldc, int64_t pitch_c,
                                   uint32_t nplanes, uint32_t slices, const PlaneConsts& consts, hipStream_t stream) {
  // the kernel moves 16-byte chunks of the workspace and of C's planes
  if (!ws || !c || m <= 0 || ldc <= 0 || ldc % 16 != 0 || pitch_c < m * ldc || pitch_c % 16 != 0 || slices == 0 ||
      nplanes == 0 || nplanes > kMaxPrefix || (reinterpret_cast<uintptr_t>(ws) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(c) & 15u) != 0)
    return hipErrorInvalidValue;
  const int64_t chunks = static_cast<int64_t>(nplanes) * m * ldc / 16;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((chunks + 31) / 32, 4096));
  hipLaunchKernelGGL(residue_finalize_kernel<8>, dim3(blocks), dim3(256), 0, stream, ws, c, m, ldc, pitch_c, nplanes,
                     slices, consts);
  return hipGetLastError();
}

}  // namespace rns8x
