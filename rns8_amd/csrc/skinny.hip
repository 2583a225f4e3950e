// Plane GEMM for results at most 16 columns wide (GEMV-like and tiny
// products) on gfx950: C_p = center(A_p x B_p mod m_p) for every residue
// plane p (reference semantics src/cpu/cpu_reference.cpp:156-206). The
// reference runs these shapes in its dedicated N <= 8 GEMV kernel
// (src/backend_hip_direct/hip_direct_gemm_tiled_kernels.cuh:298-432) and its
// M*N <= 64 persistent-small kernel (hip_direct_gemm_kernels.cuh:10-35,
// chosen at hip_backend_gemm_rns.inc:85-143).
//
// Such products are bound by reading A's planes: each A byte meets at most 16
// B columns, so the MFMA work per byte is small and the kernel is written to
// keep HBM busy rather than the matrix cores.
//   * unit = 16 * RB rows of one plane over one K slice, owned by one wave;
//     a workgroup is 4 independent waves (no barriers), each with its own
//     LDS region.
//   * MFMA: v_mfma_i32_16x16x64_i8 with the B^T fragment as src0 and the A
//     fragment as src1, so lane l ends with columns 4(l/16) .. +3 of row
//     l % 16: one packed dword of residues per lane and row block.
//   * A goes straight from HBM into registers: lane l loads 16 K-contiguous
//     bytes of row l % 16 at K offset 16 (l / 16) of each 64-K MFMA step (16
//     rows x 64 contiguous bytes per load instruction), one step ahead of
//     the MFMAs. Buffer loads read zero past the valid rows. A is read
//     exactly once, so its loads are non-temporal (8192 x 1 x 8192 at 9
//     planes: 193 -> 181 us in a step after the pack).
//   * B (16-byte rows, the plane layout) is loaded two steps ahead into
//     registers, written to the wave's LDS region one step ahead, and read
//     column-wise by ds_read_b64_tr_b8 (LDS transpose read), giving the same
//     16 K values per lane as the A fragment. B rows past the slice's K read
//     zero, which also cancels whatever A holds there.
//   * Accumulators start at 2^31 and end as u = 2^31 + sum (|sum| < 2^30 for
//     slices of at most 65536 K); the epilogue reduces with the shared byte
//     dot product + 24-bit quotient and stores 4 residues per lane.
//   * K split: when rows x planes give too few waves to keep enough loads in
//     flight, K is cut into slices whose centered residues go to an int8
//     workspace [slice][plane][M][16]; residue_finalize (fused.hip) adds them.
#include <algorithm>

#include "dma.hpp"
#include "int_ops.hpp"
#include "kernels.hpp"

namespace rns8x {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i lds_v2i;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kU = 4;                   // 64-K MFMA steps per pipeline step
constexpr int kStepK = 64 * kU;         // K per pipeline step
constexpr int kBufBytes = kStepK * 16;  // one step of B: kStepK rows x 16 bytes
constexpr int kAccBias = static_cast<int>(0x80000000u);
constexpr int kNonTemporal = 2;  // buffer-load cache policy bit: nt (streaming)
// Waves a launch aims for before it splits K (four per SIMD), and the least
// a wave streams (A rows and B's 16-byte rows of its slice), so the pipeline
// prologue stays a small share: at 8192 x 1 x 8192 (9 planes) two slices of
// 4096 run 136 us against 147 us unsplit; at 8 x 8 x 2^20, 228 slices of
// 4608 K run 45 us, 256 of 4096 K 50 us and 456 of 2304 K 55 us.
constexpr int64_t kTargetWaves = 4096;
constexpr int64_t kMinWaveBytes = 112 << 10;

struct SkinnyArgs {
  const int8_t* a;  // [planes][m][lda]
  const int8_t* b;  // [planes][k][16]
  int8_t* dst;      // C [planes][m][16] (slices == 1) or the workspace [slices][planes][m][16]
  uint32_t m, k, lda;
  uint64_t pitch_a, pitch_b, pitch_dst;  // plane pitches (bytes)
  uint32_t nplanes, groups, units;       // groups: row groups per plane
  uint32_t k_slice;
  uint32_t slices;
};

// B stage row r (16 bytes) sits at byte 16 r ^ 128 ((r >> 4) & 1): the four
// 16-row groups a transpose read touches then fall on both halves of the
// banks.
__device__ __forceinline__ int b_swz(int r) { return (r * 16) ^ (((r >> 4) & 1) << 7); }

template <int RB>
__global__ __launch_bounds__(kThreads) void skinny_gemm_kernel(SkinnyArgs a, PlaneConsts pc) {
  __shared__ __attribute__((aligned(16))) int8_t lds[kWaves][2][kBufBytes];
  const int lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t unit = blockIdx.x * kWaves + wave;
  if (unit >= a.units) return;  // whole waves leave; nothing below synchronises the workgroup
  const uint32_t group = unit % a.groups;
  const uint32_t rest = unit / a.groups;
  const uint32_t plane = rest % a.nplanes;
  const uint32_t slice = rest / a.nplanes;
  const uint32_t row0 = group * (16u * RB);
  const uint32_t rows = min(16u * RB, a.m - row0);
  const uint32_t kbeg = slice * a.k_slice;
  const uint32_t kend = min(a.k, kbeg + a.k_slice);
  const uint32_t steps = (kend - kbeg + kStepK - 1) / kStepK;

  // A: rows [row0, row0 + rows) of the plane from K offset kbeg on; the
  // resource moves kStepK bytes per step (the last step's bytes past the
  // valid rows read zero, bytes past kend meet zero B rows)
  const int8_t* const a_panel = a.a + plane * a.pitch_a + static_cast<uint64_t>(row0) * a.lda + kbeg;
  const uint32_t a_bytes = rows * a.lda - kbeg;
  // B: k rows [kbeg, kend) of the plane, 16 bytes each
  const int8_t* const b_slab = a.b + plane * a.pitch_b + static_cast<uint64_t>(kbeg) * 16u;
  const uint32_t b_bytes = (kend - kbeg) * 16u;

  const int frow = lane & 15;  // fragment row (A) / column (B)
  const int fk = lane >> 4;    // 16-K chunk of a 64-K MFMA step
  uint32_t a_off[RB][kU];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int u = 0; u < kU; ++u)
      a_off[rb][u] = static_cast<uint32_t>(16 * rb + frow) * a.lda + static_cast<uint32_t>(64 * u + 16 * fk);

  struct AFrag {
    v4i v[RB][kU];
  };
  struct BRows {
    v4i v[kU];
  };
  // past the last step the resources are empty and every lane reads zero
  auto load_a = [&](uint32_t s) {
    const bool live = s < steps;
    const __amdgpu_buffer_rsrc_t r =
        make_rsrc(a_panel + (live ? s * kStepK : 0u), live ? a_bytes - s * kStepK : 0u);
    AFrag f;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int u = 0; u < kU; ++u)
        f.v[rb][u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(a_off[rb][u]), 0, kNonTemporal));
    return f;
  };
  // lane l loads B row 64u + l of the step
  auto load_b = [&](uint32_t s) {
    const bool live = s < steps;
    const __amdgpu_buffer_rsrc_t r =
        make_rsrc(b_slab + (live ? s * kBufBytes : 0u), live ? b_bytes - s * kBufBytes : 0u);
    BRows f;
#pragma unroll
    for (int u = 0; u < kU; ++u)
      f.v[u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (64 * u + lane) * 16, 0, 0));
    return f;
  };
  int8_t* const my = &lds[wave][0][0];
  auto store_b = [&](const BRows& f, uint32_t s) {
    int8_t* const buf = my + (s & 1u) * kBufBytes;
#pragma unroll
    for (int u = 0; u < kU; ++u) *reinterpret_cast<v4i*>(buf + b_swz(64 * u + lane)) = f.v[u];
  };
  // B^T fragment of MFMA step u: in each 16-lane group (chunk fk), lane j
  // addresses the 8 bytes of row 64u + 16fk + 8h + (j >> 1), columns
  // 8 (j & 1) .. +7, and receives column j across those 8 rows.
  auto read_b = [&](uint32_t s, int u) {
    const int8_t* const buf = my + (s & 1u) * kBufBytes;
    const int r = 64 * u + 16 * fk + (frow >> 1);
    const int c = 8 * (frow & 1);
    const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(const_cast<int8_t*>(buf + (b_swz(r) | c))));
    const v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(const_cast<int8_t*>(buf + (b_swz(r + 8) | c))));
    return v4i{lo[0], lo[1], hi[0], hi[1]};
  };

  v4i acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb] = v4i{kAccBias, kAccBias, kAccBias, kAccBias};

  // Pipeline: at step s the A fragments of s are in registers, B of s is in
  // LDS buffer s & 1 and B of s + 1 in registers; step s issues the loads of
  // A(s + 1) and B(s + 2), computes s, and writes B(s + 1) to the other
  // buffer (read last at step s - 1, whose reads have completed: their
  // results fed that step's MFMAs). Steps run in pairs with the register
  // sets swapping roles, so no copy waits for a load in flight; an odd step
  // count gets one step past the end, whose loads read zero and add nothing.
  // The scheduling barriers keep the step's loads ahead of everything that
  // waits on older ones (the LDS write of B(s + 1) hoisted above them would
  // wait for every load in flight before the next ones issue).
  auto step = [&](uint32_t s, const AFrag& fa, AFrag& fa_next, const BRows& nb, BRows& nb_next) {
    fa_next = load_a(s + 1);
    nb_next = load_b(s + 2);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const v4i fb = read_b(s, u);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb, fa.v[rb][u], acc[rb], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    store_b(nb, s + 1);
  };
  AFrag fa0 = load_a(0), fa1;
  store_b(load_b(0), 0);
  BRows nb0 = load_b(1), nb1;
  for (uint32_t s = 0; s < steps; s += 2) {
    step(s, fa0, fa1, nb0, nb1);
    step(s + 1, fa1, fa0, nb1, nb0);
  }

  // Epilogue: lane l holds u = 2^31 + C[row0 + 16 rb + l % 16][4 (l / 16) + e]
  // in element e of acc[rb].
  const ModulusConsts mc = pc.mod[plane];
  const CenteredI32 kc = centered_i32_consts(mc);
  int8_t* const dst = a.dst + (static_cast<uint64_t>(slice) * a.nplanes + plane) * a.pitch_dst;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const uint32_t row = row0 + 16u * rb + static_cast<uint32_t>(frow);
    uint32_t r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = centered_residue_i32(static_cast<uint32_t>(acc[rb][e]), mc, kc);
    if (row < a.m)
      *reinterpret_cast<uint32_t*>(dst + static_cast<uint64_t>(row) * 16u + 4u * fk) =
          pack_low_bytes(r[0], r[1], r[2], r[3]);
  }
}

// Row blocks per wave: 32 rows halve B's LDS traffic per A byte against 16;
// 64 rows ran slower (156 against 145 us at 8192 x 1 x 8192) and need 224
// registers.
int rows_per_wave_blocks(int64_t m) { return m <= 16 ? 1 : 2; }

}  // namespace

bool skinny_shape(int64_t m, int64_t n, int64_t k, uint32_t nplanes, GemmShape& out) {
  if (n > 16 || m <= 0 || n <= 0 || k <= 0 || nplanes == 0) return false;
  const int rb = rows_per_wave_blocks(m);
  const int64_t waves = (m + 16 * rb - 1) / (16 * rb) * nplanes;
  // slices of at most 65536 K (int32-exact), toward kTargetWaves waves that
  // each stream at least kMinWaveBytes
  const int64_t need = (k + kSafeKBlock - 1) / kSafeKBlock;
  const int64_t wave_bytes = k * (std::min<int64_t>(m, 16 * rb) + 16);
  int64_t slices = std::min((kTargetWaves + waves - 1) / waves, std::max<int64_t>(1, wave_bytes / kMinWaveBytes));
  slices = std::max(slices, need);
  int64_t k_slice = (k + slices - 1) / slices;
  if (slices > 1) k_slice = (k_slice + kStepK - 1) / kStepK * kStepK;
  slices = (k + k_slice - 1) / k_slice;
  if (waves * slices > 0x7FFFFFFF) return false;
  out.tile = 16;
  out.slices = static_cast<uint32_t>(slices);
  out.k_slice = k_slice;
  out.ws_bytes = slices > 1 ? static_cast<uint64_t>(slices) * nplanes * static_cast<uint64_t>(m) * 16u : 0u;
  return true;
}

hipError_t launch_skinny(const GemmArgs& g, const GemmShape& shape, const PlaneConsts& consts, hipStream_t stream) {
  // shape limits: 16-byte B and C rows, 32-bit offsets inside a row panel
  if (g.ldb != 16 || g.ldc != 16 || shape.tile != 16 || g.lda >= (int64_t{1} << 23) || g.k >= (int64_t{1} << 31))
    return hipErrorInvalidValue;
  if (shape.slices > 1 && !g.splitk_ws) return hipErrorInvalidValue;
  const int rb = rows_per_wave_blocks(g.m);
  SkinnyArgs a{};
  a.a = g.a;
  a.b = g.b;
  a.m = static_cast<uint32_t>(g.m);
  a.k = static_cast<uint32_t>(g.k);
  a.lda = static_cast<uint32_t>(g.lda);
  a.pitch_a = static_cast<uint64_t>(g.pitch_a);
  a.pitch_b = static_cast<uint64_t>(g.pitch_b);
  a.nplanes = g.nplanes;
  a.groups = static_cast<uint32_t>((g.m + 16 * rb - 1) / (16 * rb));
  a.slices = shape.slices;
  a.k_slice = static_cast<uint32_t>(shape.slices > 1 ? shape.k_slice : g.k);
  const uint64_t units = static_cast<uint64_t>(a.groups) * g.nplanes * shape.slices;
  if (units == 0 || units > 0x7FFFFFFFull) return hipErrorInvalidValue;
  a.units = static_cast<uint32_t>(units);
  if (shape.slices > 1) {
    a.dst = g.splitk_ws;
    a.pitch_dst = static_cast<uint64_t>(g.m) * 16u;
  } else {
    a.dst = g.c;
    a.pitch_dst = static_cast<uint64_t>(g.pitch_c);
  }
  const dim3 grid(static_cast<unsigned>((units + kWaves - 1) / kWaves));
  if (rb == 1)
    hipLaunchKernelGGL(skinny_gemm_kernel<1>, grid, dim3(kThreads), 0, stream, a, consts);
  else
    hipLaunchKernelGGL(skinny_gemm_kernel<2>, grid, dim3(kThreads), 0, stream, a, consts);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || shape.slices <= 1) return e;
  return launch_residue_finalize(g.splitk_ws, g.c, g.m, 16, g.pitch_c, g.nplanes, shape.slices, consts, stream);
}

}  // namespace rns8x
