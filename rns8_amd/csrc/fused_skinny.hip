// Fused native-input GEMM for results at most 16 columns wide (GEMV and
// tall-skinny products): C's residue planes straight from int64 / uint64
// device operands, A's residues formed in registers and never stored
// (reference hip_direct_gemm_native_kernels.cuh:9-193 converts native
// operands inside its tile loads; its N <= 8 GEMV is
// hip_direct_gemm_tiled_kernels.cuh:298-432).
//
// The packed route writes every residue plane of A to HBM and reads it back:
// at 8192 x 1 x 8192 with 9 planes that is 537 MB read, 604 MB written and
// 604 MB read again. Here A's 537 MB are read once and each element is
// reduced once per plane in registers, so the pass is bound by that read and
// by the reduction's VALU work, which are about equal on MI355X.
//
// Work split: a wave owns 16 rows of A, one K slice and up to kMaxGroup
// planes, so A is loaded once for all of them (results of more than 18
// planes run two plane groups, each loading A; 8192 x 1 x 8192: 150 us at 9
// planes, 177 at 12, 219 at 16, 245 at 18, 322 at 20 in two groups; with at
// most 9 planes per wave 12 planes took 245 us, and 20 planes in one group,
// which spills inside the loop, 676 us). The loads are what bounds the pass: with the planes spread
// over three waves per row block (162 registers, three waves per SIMD) in the
// hope that the other waves find A in L2, each wave's loads cost as much as
// the first one's (358 against 187 us at 9 planes).
//   * A: a 64-K step of the wave's 16 rows is eight 16-byte loads per lane,
//     one step ahead (ordinary loads: the two halves of a 128-byte line
//     come from consecutive loads, and non-temporal ones were 4% slower): load j of lane l reads elements
//     8j + 2 (l / 16) and +1 of row l % 16, so each load instruction covers
//     64 contiguous bytes of every row (with the 16 K-contiguous elements per
//     lane that the MFMA layout suggests, it touched 64 cache lines and ran
//     1.6x slower). The dot product does not depend on the order of K, so
//     the MFMA's K slot 16 (l / 16) + e of the step holds element
//     8 (e / 2) + 2 (l / 16) + e % 2, and B's planes are stored in the same
//     order. Rows past m and elements past the operand's last logical element
//     read zero through the buffer range.
//   * Conversion: per plane the 16 elements reduce to centered residue
//     bytes (the pack's arithmetic: two byte dot products and a 24-bit
//     quotient, one dot product when every element of the wave's step fits
//     in 32 bits), which form the lane's A fragment of
//     v_mfma_i32_16x16x64_i8 directly: lane l holds row l % 16, K 16 (l / 16)
//     .. +15, one byte each.
//   * B: a small kernel first writes B's residue planes into the workspace
//     as [plane][64-K step][16 columns][64 K slots] in that K order, with
//     zeros past K and past n, so the B^T fragment of a plane (column l % 16,
//     the lane's 16 K slots) is one 16-byte load from L2, also one step
//     ahead, and a wave's load covers 1 KB of contiguous bytes. Zero B past K
//     cancels whatever A holds there.
//   * Accumulators start at 2^31 (slices of at most 65536 K keep the sum
//     exact); the epilogue reduces like the skinny kernel's and stores one
//     packed dword of residues per lane and plane, into C's planes or, with
//     K split, into the int8 slot of the slice ([slice][plane][m][16]) that
//     residue_finalize adds up.
#include <algorithm>
#include <type_traits>

#include "dma.hpp"
#include "int_ops.hpp"
#include "kernels.hpp"

namespace rns8x {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kStep = 64;           // K per MFMA step
constexpr int kMaxGroup = 18;       // planes per wave (243 registers at 16; 17 and 18 spill a few, 20 many)
constexpr int kMinBlocks = 2;       // workgroups per CU (256 registers)
constexpr int kAccBias = static_cast<int>(0x80000000u);
constexpr int64_t kTargetWaves = 4096;
constexpr int64_t kMinSliceK = 1024;  // 16 steps per wave at least, unless K is shorter
constexpr int64_t kMaxK = int64_t{1} << 23;
// B's transposed planes take P x 16 bytes per k: 256 MiB admits 8 x 8 x 2^20 at 9 planes (151 MB), where the
// tile form would convert B's 8 columns as 128
constexpr uint64_t kMaxWorkspace = uint64_t{256} << 20;

struct SkinnyFusedArgs {
  const uint64_t* a;  // native A, m x k at row stride lda (elements)
  uint32_t lda, m, k, kp;
  const int8_t* bt;   // [nplanes][16][kp] transposed B planes
  int8_t* dst;        // C's planes (one slice) or the residue slots
  uint64_t pitch_dst; // bytes between consecutive planes of dst
  uint32_t nplanes;   // planes of the result (slot layout)
  uint32_t plane0;    // the launch's first plane
  uint32_t row_blocks, units, k_slice;  // units: workgroups (4 row blocks of one slice)
};

// Centered residue of the 64-bit value (hi:lo) mod mc.m (pack.hip's wide
// form; a signed value is read as x ^ 2^63, the bias folded into off_i64).
template <bool Signed>
__device__ __forceinline__ uint32_t residue64(uint32_t lo, uint32_t hi, const ModulusConsts& mc) {
  if (mc.m == 256u) return lo;
  const uint32_t off = (Signed ? mc.off_i64 : mc.off_u64) - mc.half;
  const uint32_t t = __builtin_amdgcn_udot4(lo, mc.pow_lo, off, false);
  const uint32_t s = __builtin_amdgcn_udot4(Signed ? hi ^ 0x80000000u : hi, mc.pow_hi, t, false);
  return centered_byte(s, mc.pq_shift, in_vgpr(mc.half << mc.pq_shift), mc.pq_recip, 256u - mc.m);
}

// B^T planes: thread t of grid row p writes byte run t (16 bytes) of plane p
// (one plane per grid row, so even a small B spreads over the chip): K slots
// 16q .. 16q + 15 of column c in 64-K step s, t = 64 s + 4 c + q; slot
// 16q + e holds k = 64 s + 8 (e / 2) + 2q + e % 2 (the order of the A loads);
// columns past n and k past K are zero.
template <bool Signed>
__global__ __launch_bounds__(256) void pack_bt_kernel(const uint64_t* b, int64_t ldb, uint32_t k, uint32_t n,
                                                      uint32_t kp, int8_t* bt, PlaneConsts pc) {
  const uint32_t runs = kp / 16u;
  const uint32_t total = 16u * runs;
  for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < total; t += gridDim.x * blockDim.x) {
    // t = (step, column, quarter) with the quarter fastest: consecutive
    // threads write consecutive 16-byte runs
    const uint32_t fq = t & 3u, col = (t >> 2) & 15u, kb = (t >> 6) * 64u;
    uint32_t lo[16], hi[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t ke = kb + 8u * (e >> 1) + 2u * fq + (e & 1);
      const uint64_t x = (col < n && ke < k) ? b[static_cast<int64_t>(ke) * ldb + col] : 0ull;
      lo[e] = static_cast<uint32_t>(x);
      hi[e] = static_cast<uint32_t>(x >> 32);
    }
    const uint32_t p = blockIdx.y;
    const ModulusConsts mc = pc.mod[p];
    uint32_t r[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) r[e] = residue64<Signed>(lo[e], hi[e], mc);
    const v4i w = v4i{static_cast<int>(pack_low_bytes(r[0], r[1], r[2], r[3])),
                      static_cast<int>(pack_low_bytes(r[4], r[5], r[6], r[7])),
                      static_cast<int>(pack_low_bytes(r[8], r[9], r[10], r[11])),
                      static_cast<int>(pack_low_bytes(r[12], r[13], r[14], r[15]))};
    *reinterpret_cast<v4i*>(bt + static_cast<uint64_t>(p) * 16u * kp + static_cast<uint64_t>(t) * 16u) = w;
  }
}

// A lane's eight 16-byte loads of one step: element e (K slot 16 (l / 16) + e
// of the step, k = 8 (e / 2) + 2 (l / 16) + e % 2) is v[e / 2][2 (e % 2)] (low
// half) and v[e / 2][2 (e % 2) + 1] (high half).
struct Raw {
  v4i v[8];
};
// The workgroup's share of one step's B planes: 16-byte chunks t, t + 256,
// t + 512 of the G KB (thread t).
constexpr int kBChunksPerThread = (kMaxGroup * 64 + kThreads - 1) / kThreads;
struct BChunks {
  v4i v[kBChunksPerThread];
};

// One launch per group of G planes, plane0 .. plane0 + G - 1. A workgroup
// is four consecutive row blocks (one per wave) of one K slice, so its waves
// share each step's B fragments: the workgroup loads them into LDS once (a
// step of B is G KB), double-buffered with one barrier per step. Waves past
// the last row block run the loop with empty loads and store nothing.
// kFirst256: the group holds plane 0, the ladder's m = 256.
template <bool Signed, int G, bool kFirst256>
__global__ __launch_bounds__(kThreads, kMinBlocks) void fused_skinny_kernel(SkinnyFusedArgs a, PlaneConsts pc) {
  __shared__ __attribute__((aligned(16))) int8_t bsh[2][G * 1024];
  const int lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t quads = (a.row_blocks + kWaves - 1) / kWaves;
  const uint32_t slice = blockIdx.x / quads;
  const uint32_t rb = (blockIdx.x - slice * quads) * kWaves + wave;
  const uint32_t p0 = a.plane0;
  const uint32_t row0 = rb * 16u;
  const uint32_t rows = rb < a.row_blocks ? min(16u, a.m - row0) : 0u;
  const uint32_t kbeg = slice * a.k_slice;
  const uint32_t kend = min(a.k, kbeg + a.k_slice);
  const uint32_t steps = (kend - kbeg + kStep - 1) / kStep;
  const int frow = lane & 15;  // fragment row (A) / column (B)
  const int fk = lane >> 4;    // 16-K chunk of a step

  // A: the step's resource starts at its first k in row row0 and ends at the
  // operand's last logical element of the wave's rows (a row past them lies
  // beyond it, since lda >= k); past the last step it is empty
  const uint64_t* const a_rows = a.a + static_cast<uint64_t>(row0) * a.lda;
  const uint32_t a_lane = (static_cast<uint32_t>(frow) * a.lda + 2u * fk) * 8u;
  auto load_a = [&](uint32_t s, Raw& x) {
    const bool live = s < steps && rows > 0u;
    const uint32_t k0 = kbeg + (live ? s : 0u) * kStep;
    const int64_t bytes = live ? (static_cast<int64_t>(rows - 1) * a.lda + (a.k - k0)) * 8 : 0;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(a_rows + k0, bytes);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      x.v[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(a_lane + 64u * j),
                                                                              0, 0));
  };
  // B: chunk q (16 bytes) of a step is column c = (q % 64) / 4, K slots
  // 16 (q % 4) .. +15 of plane p0 + q / 64. In LDS it sits at 16 (64 (q / 64)
  // + 4c + (q % 4 ^ (c / 4) % 4)): a fragment read (16 lanes, columns 0-15,
  // one slot quarter) then covers 16 distinct bank quads. Past the last step
  // the first step's chunks are read again and meet zero A.
  const int8_t* const bt_group = a.bt + static_cast<uint64_t>(p0) * 16u * a.kp;
  auto load_b = [&](uint32_t s, BChunks& f) {
    const uint32_t k0 = kbeg + (s < steps ? s : 0u) * kStep;
#pragma unroll
    for (int i = 0; i < kBChunksPerThread; ++i) {
      const uint32_t q = threadIdx.x + kThreads * i;
      if (q < G * 64u)
        f.v[i] = *reinterpret_cast<const v4i*>(bt_group + static_cast<uint64_t>(q >> 6) * 16u * a.kp + 16u * k0 +
                                               16u * (q & 63u));
    }
  };
  auto lds_pos = [](uint32_t q) {
    const uint32_t c = (q & 63u) >> 2;
    return 16u * (64u * (q >> 6) + 4u * c + ((q & 3u) ^ ((c >> 2) & 3u)));
  };
  auto store_b = [&](const BChunks& f, int stage) {
#pragma unroll
    for (int i = 0; i < kBChunksPerThread; ++i) {
      const uint32_t q = threadIdx.x + kThreads * i;
      if (q < G * 64u) *reinterpret_cast<v4i*>(&bsh[stage][lds_pos(q)]) = f.v[i];
    }
  };
  // this lane's fragment of plane p: column frow, slot quarter fk
  const uint32_t frag_pos = lds_pos(static_cast<uint32_t>(4 * frow + fk));
  auto read_b = [&](int stage, int p) { return *reinterpret_cast<const v4i*>(&bsh[stage][1024 * p + frag_pos]); };

  v4i acc[G];
#pragma unroll
  for (int p = 0; p < G; ++p) acc[p] = v4i{kAccBias, kAccBias, kAccBias, kAccBias};

  // One plane's A fragment from the step's 16 elements, then its MFMA. kFast:
  // every element of the wave fits 32 bits (int32 / uint32), and lo holds
  // the low words (x ^ 2^31 for signed input, read by the int32 reduction);
  // otherwise lo and hi are the two words (hi ^ 2^31 for signed input). kM256:
  // the ladder's first modulus, 256, whose centered residue is the low byte
  // (unchanged by the bias). A step's planes are straight-line code, so the
  // constants' scalar loads issue early.
  auto plane_mma = [&](auto fast, auto m256, const uint32_t (&lo)[16], const uint32_t (&hi)[16], int stage, int p,
                       v4i& acc_p, const ModulusConsts& mc) {
    constexpr bool kFast = decltype(fast)::value;
    v4i fa;
    if constexpr (decltype(m256)::value) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        fa[q] = static_cast<int>(pack_low_bytes(lo[4 * q], lo[4 * q + 1], lo[4 * q + 2], lo[4 * q + 3]));
    } else {
      constexpr bool kI32 = kFast && Signed;
      const uint32_t shift = kI32 ? mc.q_shift : mc.pq_shift;
      const uint32_t recip = kI32 ? mc.q_recip : mc.pq_recip;
      const uint32_t off = (kI32 ? mc.off_i32 : Signed ? mc.off_i64 : mc.off_u64) - mc.half;
      const uint32_t h_sh = in_vgpr(mc.half << shift), m_comp = 256u - mc.m;
      // four residues at a time, packed as soon as they are formed
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint32_t sv = __builtin_amdgcn_udot4(lo[4 * q + e], mc.pow_lo, off, false);
          if constexpr (!kFast) sv = __builtin_amdgcn_udot4(hi[4 * q + e], mc.pow_hi, sv, false);
          r[e] = centered_byte(sv, shift, h_sh, recip, m_comp);
        }
        fa[q] = static_cast<int>(pack_low_bytes(r[0], r[1], r[2], r[3]));
      }
    }
    acc_p = __builtin_amdgcn_mfma_i32_16x16x64_i8(read_b(stage, p), fa, acc_p, 0, 0, 0);
  };

  {
    auto planes = [&](auto fast, const uint32_t (&lo)[16], const uint32_t (&hi)[16], int stage) {
#pragma unroll
      for (int p = 0; p < G; ++p) {
        if (kFirst256 && p == 0)
          plane_mma(fast, std::true_type{}, lo, hi, stage, p, acc[p], pc.mod[0]);
        else
          plane_mma(fast, std::false_type{}, lo, hi, stage, p, acc[p], pc.mod[p0 + p]);
      }
    };
    auto compute = [&](const Raw& x, int stage) {
      uint32_t lo[16], hi[16];
      uint32_t wide = 0;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        lo[e] = static_cast<uint32_t>(x.v[e >> 1][2 * (e & 1)]);
        hi[e] = static_cast<uint32_t>(x.v[e >> 1][2 * (e & 1) + 1]);
        wide |= Signed ? hi[e] ^ static_cast<uint32_t>(static_cast<int32_t>(lo[e]) >> 31) : hi[e];
      }
      // one branch per wave and step; the signed bias is applied once per
      // element, not once per plane
      if (__builtin_amdgcn_ballot_w64(wide != 0u) == 0u) {
        if constexpr (Signed) {
#pragma unroll
          for (int e = 0; e < 16; ++e) lo[e] ^= 0x80000000u;
        }
        planes(std::true_type{}, lo, hi, stage);
      } else {
        if constexpr (Signed) {
#pragma unroll
          for (int e = 0; e < 16; ++e) hi[e] ^= 0x80000000u;
        }
        planes(std::false_type{}, lo, hi, stage);
      }
    };
    // Steps run in pairs with the register sets swapping roles, so no copy
    // waits for a load in flight; an odd step count gets one step past the
    // end, whose A reads zero and adds nothing. Step s reads B from LDS
    // stage s & 1 while the chunks of step s + 1 arrive in registers (loaded
    // before A, so waiting for them leaves A's loads in flight); they go to
    // the other stage, whose readers finished before the previous barrier,
    // and the barrier after the write publishes them.
    Raw x0, x1;
    BChunks nb;
    load_b(0, nb);
    load_a(0, x0);
    store_b(nb, 0);
    __syncthreads();
    for (uint32_t s = 0; s < steps; s += 2) {
      load_b(s + 1, nb);
      load_a(s + 1, x1);
      __builtin_amdgcn_sched_barrier(0);
      compute(x0, 0);
      __builtin_amdgcn_sched_barrier(0);
      store_b(nb, 1);
      __syncthreads();
      load_b(s + 2, nb);
      load_a(s + 2, x0);
      __builtin_amdgcn_sched_barrier(0);
      compute(x1, 1);
      __builtin_amdgcn_sched_barrier(0);
      store_b(nb, 0);
      __syncthreads();
    }
  }

  // Epilogue: lane l holds u = 2^31 + C[row0 + l % 16][4 (l / 16) + e] in
  // element e of acc[p].
  const uint32_t row = row0 + static_cast<uint32_t>(frow);
#pragma unroll
  for (int p = 0; p < G; ++p) {
    const ModulusConsts mc = pc.mod[p0 + p];
    const CenteredI32 kc = centered_i32_consts(mc);
    uint32_t r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = centered_residue_i32(static_cast<uint32_t>(acc[p][e]), mc, kc);
    int8_t* const dst = a.dst + (static_cast<uint64_t>(slice) * a.nplanes + p0 + p) * a.pitch_dst;
    if (rows > 0u && row < a.m)
      *reinterpret_cast<uint32_t*>(dst + static_cast<uint64_t>(row) * 16u + 4u * fk) =
          pack_low_bytes(r[0], r[1], r[2], r[3]);
  }
}

template <bool Signed, int G>
void launch_planes(const SkinnyFusedArgs& a, const PlaneConsts& consts, hipStream_t stream) {
  const dim3 grid(a.units);
  if (a.plane0 == 0)
    hipLaunchKernelGGL((fused_skinny_kernel<Signed, G, true>), grid, dim3(kThreads), 0, stream, a, consts);
  else
    hipLaunchKernelGGL((fused_skinny_kernel<Signed, G, false>), grid, dim3(kThreads), 0, stream, a, consts);
}

// Planes of group g of the result's nplanes: at most kMaxGroup, the groups
// as even as possible.
uint32_t groups_of(uint32_t nplanes) { return (nplanes + kMaxGroup - 1) / kMaxGroup; }
uint32_t group_planes(uint32_t nplanes, uint32_t g) {
  const uint32_t groups = groups_of(nplanes);
  return nplanes / groups + (g < nplanes % groups ? 1u : 0u);
}

int64_t kp_of(int64_t k) { return (k + kStep - 1) / kStep * kStep; }

}  // namespace

bool fused_skinny_shape(int64_t m, int64_t n, int64_t k, uint32_t nplanes, FusedShape& out) {
  out = FusedShape{};
  if (n <= 0 || n > 16 || m <= 0 || k <= 0 || nplanes == 0 || nplanes > kMaxPrefix) return false;
  if (m >= (int64_t{1} << 31) || k > kMaxK) return false;
  const int64_t waves = (m + 15) / 16;
  // toward kTargetWaves waves, slices of at least kMinSliceK and at most
  // 65536 K (int32-exact); split slices are whole steps
  int64_t slices = std::min((kTargetWaves + waves - 1) / waves, (k + kMinSliceK - 1) / kMinSliceK);
  slices = std::max(std::max<int64_t>(slices, 1), (k + kSafeKBlock - 1) / kSafeKBlock);
  int64_t k_slice = (k + slices - 1) / slices;
  if (slices > 1) k_slice = (k_slice + kStep - 1) / kStep * kStep;
  slices = (k + k_slice - 1) / k_slice;
  if (waves * slices > 0x7FFFFFFF || slices > 65535) return false;
  const uint64_t bt = static_cast<uint64_t>(nplanes) * 16u * static_cast<uint64_t>(kp_of(k));
  const uint64_t slots = slices > 1 ? static_cast<uint64_t>(slices) * nplanes * static_cast<uint64_t>(m) * 16u : 0u;
  if (bt + slots > kMaxWorkspace) return false;
  out.slices = static_cast<uint32_t>(slices);
  out.k_slice = k_slice;
  out.ws_bytes = bt + slots;
  out.skinny = 1;
  out.bt_bytes = bt;
  return true;
}

hipError_t launch_fused_skinny(const FusedArgs& f, const PlaneConsts& consts, hipStream_t stream) {
  const FusedShape& sh = f.shape;
  if (!sh.skinny || f.ldc != 16 || f.n > 16 || f.k > kMaxK || f.lda >= (int64_t{1} << 21)) return hipErrorInvalidValue;
  const int64_t kp = kp_of(f.k);
  const bool sgn = f.kind == NativeKind::I64;
  // B's transposed residue planes at the start of the workspace
  const uint32_t runs_total = static_cast<uint32_t>(kp);  // 16 columns x kp / 16 runs
  const dim3 bt_blocks(static_cast<unsigned>(std::min<int64_t>((runs_total + 255) / 256, 8192)), f.nplanes);
  if (sgn)
    hipLaunchKernelGGL(pack_bt_kernel<true>, bt_blocks, dim3(256), 0, stream,
                       static_cast<const uint64_t*>(f.b), f.ldb, static_cast<uint32_t>(f.k),
                       static_cast<uint32_t>(f.n), static_cast<uint32_t>(kp), f.ws, consts);
  else
    hipLaunchKernelGGL(pack_bt_kernel<false>, bt_blocks, dim3(256), 0, stream,
                       static_cast<const uint64_t*>(f.b), f.ldb, static_cast<uint32_t>(f.k),
                       static_cast<uint32_t>(f.n), static_cast<uint32_t>(kp), f.ws, consts);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;

  SkinnyFusedArgs a{};
  a.a = static_cast<const uint64_t*>(f.a);
  a.lda = static_cast<uint32_t>(f.lda);
  a.m = static_cast<uint32_t>(f.m);
  a.k = static_cast<uint32_t>(f.k);
  a.kp = static_cast<uint32_t>(kp);
  a.bt = f.ws;
  a.nplanes = f.nplanes;
  a.row_blocks = static_cast<uint32_t>((f.m + 15) / 16);
  a.k_slice = static_cast<uint32_t>(sh.slices > 1 ? sh.k_slice : f.k);
  int8_t* const slots = f.ws + sh.bt_bytes;
  if (sh.slices > 1) {
    a.dst = slots;
    a.pitch_dst = static_cast<uint64_t>(f.m) * 16u;
  } else {
    a.dst = f.c;
    a.pitch_dst = static_cast<uint64_t>(f.pitch_c);
  }
  a.units = (a.row_blocks + kWaves - 1) / kWaves * sh.slices;  // workgroups
  // one launch per plane group, each reading A
  uint32_t base = 0;
  for (uint32_t g = 0; g < groups_of(f.nplanes); ++g) {
    const uint32_t np = group_planes(f.nplanes, g);
    a.plane0 = base;
    auto launch = [&](auto sgn) {
      constexpr bool S = decltype(sgn)::value;
      switch (np) {
        case 1: launch_planes<S, 1>(a, consts, stream); break;
        case 2: launch_planes<S, 2>(a, consts, stream); break;
        case 3: launch_planes<S, 3>(a, consts, stream); break;
        case 4: launch_planes<S, 4>(a, consts, stream); break;
        case 5: launch_planes<S, 5>(a, consts, stream); break;
        case 6: launch_planes<S, 6>(a, consts, stream); break;
        case 7: launch_planes<S, 7>(a, consts, stream); break;
        case 8: launch_planes<S, 8>(a, consts, stream); break;
        case 9: launch_planes<S, 9>(a, consts, stream); break;
        case 10: launch_planes<S, 10>(a, consts, stream); break;
        case 11: launch_planes<S, 11>(a, consts, stream); break;
        case 12: launch_planes<S, 12>(a, consts, stream); break;
        case 13: launch_planes<S, 13>(a, consts, stream); break;
        case 14: launch_planes<S, 14>(a, consts, stream); break;
        case 15: launch_planes<S, 15>(a, consts, stream); break;
        case 16: launch_planes<S, 16>(a, consts, stream); break;
        case 17: launch_planes<S, 17>(a, consts, stream); break;
        case 18: launch_planes<S, 18>(a, consts, stream); break;
        case 19: launch_planes<S, 19>(a, consts, stream); break;
        default: launch_planes<S, 20>(a, consts, stream); break;
      }
    };
    if (sgn)
      launch(std::true_type{});
    else
      launch(std::false_type{});
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    base += np;
  }
  if (sh.slices <= 1) return hipSuccess;
  return launch_residue_finalize(slots, f.c, f.m, 16, f.pitch_c, f.nplanes, sh.slices, consts, stream);
}

}  // namespace rns8x
