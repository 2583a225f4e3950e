// Plane-batched int8 MFMA GEMM for gfx950 (CDNA4).
//
// One launch computes C_p = center(A_p x B_p mod m_p) for every residue plane
// p (reference semantics: src/cpu/cpu_reference.cpp:156-206, the per-modulus
// ring GEMM with int32 accumulation reduced at least every 65536 K).
//
// Work decomposition
//   * workgroup = 256 threads (4 wave64s) owning a 256x256 output tile of one
//     plane (and one K slice when split-K is on); waves form a 2x2 grid of
//     128x128 wave tiles.
//   * K is consumed in BK = 64 byte steps through a 4-stage LDS ring. Both
//     operands go global -> LDS by buffer-load DMA (no VGPR staging): A tiles
//     (256 x 64, K-contiguous rows) and B tiles (64 x 256, N-contiguous rows,
//     the layout they have in HBM). The DMA of step t+3 is in flight while
//     step t computes; one barrier per step.
//   * A fragments are ds_read_b128 of 16 K-contiguous bytes; B fragments are
//     gathered K-contiguous from the N-contiguous stage by ds_read_b64_tr_b8
//     (LDS transpose read), so no transpose runs on the VALU.
//   * Stage rows are XOR-swizzled in 16-byte chunks (swizzle applied on the
//     global-address side of the DMA) so every fragment read is bank-conflict
//     free.
//   * MFMA: v_mfma_i32_32x32x32_i8 with the B^T fragment as src0 and the A
//     fragment as src1, so each lane ends with 4 consecutive output columns
//     of one row per register group -> one packed dword store per group.
//   * Exactness: |a*b| <= 2^14, so <= 65536 products plus a carried residue
//     fit int32. One launch covers at most 65536 K; the host issues longer K
//     as consecutive launches whose epilogues add the residue already in C.
//   * Epilogue: accumulators start at 2^31, so each holds the biased sum the
//     reduction reads; reduction is a byte dot product plus a 24-bit
//     reciprocal quotient (full-rate VALU only), and 4 residues are packed per
//     dword store.
//   * Split-K (tall-skinny K): each slice reduces (when K > 65536) and
//     atomically adds its partial into an int32 workspace; a finalize kernel
//     reduces to int8 and clears the workspace.
#include <type_traits>

#include "int_ops.hpp"
#include "kernels.hpp"

namespace rns8x {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i lds_v2i;

__device__ __forceinline__ lds_v2i* as_lds_v2i(const int8_t* p) {
  return (lds_v2i*)(const_cast<int8_t*>(p));  // generic -> LDS address space
}
__device__ __forceinline__ uint32_t lds_address(const int8_t* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) int8_t*)(const_cast<int8_t*>(p))));
}

// s_waitcnt immediates "vmcnt <= n" leaving expcnt and lgkmcnt unconstrained
// (gfx9 encoding: vmcnt[3:0] bits 3:0, expcnt bits 6:4, lgkmcnt bits 11:8,
// vmcnt[5:4] bits 15:14).
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kWaitVm[9] = {wait_vm(0), wait_vm(1), wait_vm(2), wait_vm(3), wait_vm(4),
                            wait_vm(5), wait_vm(6), wait_vm(7), wait_vm(8)};

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kThreads = 256;
constexpr int kGroupM = 4;  // tile rows per L2 reuse group
// Buffer resource word 3 for gfx9-family raw buffers (32-bit data format).
constexpr int kBufferFlags = 0x00020000;

template <int BK>
struct Tile {
  static constexpr int kBufA = kBM * BK;              // A stage: 256 rows x BK bytes
  static constexpr int kBufB = kBN * BK;              // B stage: BK k-rows x 256 bytes
  static constexpr int kStage = kBufA + kBufB;
  static constexpr int kStages = 4;
  static constexpr int kLds = kStages * kStage;       // 128 KB of the 160 KB LDS
  static constexpr int kDma = kBufA / 1024 / 4;       // 1 KB DMA blocks per wave, per operand
};

// A stage: row-major 256 x 64 bytes. The 16-byte chunk index is XORed with
// row bits 1-5 so the ds_read_b128 fragment loads (32 consecutive rows, one
// chunk) are bank-conflict free for both 32-bank/8-lane and 64-bank/16-lane
// servicing (exhaustive host model).
__device__ __forceinline__ int swizzle_a(int row, int chunk) {
  return chunk ^ (((row >> 1) & 3) ^ (((row >> 3) & 1) * 3) ^ ((row >> 4) & 3));
}

// B stage: row-major 64 (k) x 256 (n) bytes, N-contiguous as in global
// memory. The 16-byte chunk index is XORed with f(k & 7), f(x) = 2x mod 16 +
// x / 4: a 16-lane transpose read touches 8 consecutive k rows of one chunk,
// and f sends them to 8 (32-bank model) resp., with the neighbouring group,
// 16 (64-bank model) distinct bank quads (exhaustive host model).
__device__ __forceinline__ int swizzle_b(int k, int chunk) {
  const int x = k & 7;
  return chunk ^ (((2 * x) & 15) | (x >> 2));
}

// Accumulator start value: the MFMAs then produce u = 2^31 + sum (mod 2^32),
// the biased form the reduction reads (|sum| < 2^31).
constexpr int kAccBias = static_cast<int>(0x80000000u);

// For u = x + 2^31 (x an int32 sum), returns a value whose low byte is
// (x + H) mod m, H = floor(m/2): s = dot(bytes(u), 2^(8b) mod m) + off_i32 is
// congruent to x + H and at most s_max, q = floor(s / m) by the 24-bit
// quotient of tables.hpp, and s + q*(256 - m) is congruent to s - q*m modulo
// 256. m_comp = 256 - m.
__device__ __forceinline__ uint32_t residue_plus_half(uint32_t u, const ModulusConsts& mc, uint32_t m_comp) {
  return mod_low_byte(__builtin_amdgcn_udot4(u, mc.pow_lo, mc.off_i32, false), mc.q_shift, mc.q_recip, m_comp);
}

// Raw buffer resource over [p, p + bytes). The inputs are wave-uniform; they
// are passed through readfirstlane so the descriptor is built in SGPRs.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
  const uint64_t addr = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr >> 32));
  const int n = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
  void* const base = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(base, static_cast<short>(0), n, kBufferFlags);
}

// The same resource as four wave-uniform dwords, for the DMA asm below.
__device__ __forceinline__ v4i buffer_rsrc(const void* p, int64_t bytes) {
  const uint64_t addr = reinterpret_cast<uint64_t>(p);
  return v4i{__builtin_amdgcn_readfirstlane(static_cast<int>(addr)),
             __builtin_amdgcn_readfirstlane(static_cast<int>(addr >> 32)),
             __builtin_amdgcn_readfirstlane(static_cast<int>(bytes)), kBufferFlags};
}

// 16 bytes per lane from a raw buffer straight into LDS: lane l's bytes land
// at lds_addr + 16*l (M0 = lds_addr, wave-uniform). Written as asm so the
// compiler does not track the LDS write (it would otherwise wait for every
// outstanding DMA before each LDS read); callers order the DMA against LDS
// reads with explicit vmcnt waits and barriers. M0 is a reserved register the
// compiler re-initialises before any use of its own.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(uint32_t lds_addr, uint32_t voffset, v4i rsrc) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voffset), "s"(rsrc)
               : "m0");
}
#pragma clang diagnostic pop

template <int BK>
__global__ __launch_bounds__(kThreads, 1) void plane_gemm_kernel(GemmArgs args, PlaneConsts pc, uint32_t tiles_m,
                                                                  uint32_t tiles_n, int64_t k_begin, int64_t k_stop,
                                                                  int64_t k_slice, uint32_t accumulate) {
  using T = Tile<BK>;
  static_assert(BK == 64, "fragment schedule below assumes two k32 sub-steps per K step");
  __shared__ __attribute__((aligned(16))) int8_t lds[T::kLds];

  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wave_m = wave >> 1;
  const int wave_n = wave & 1;

  // ---- block -> (slice, plane, tile) with XCD-aware ordering --------------
  // Workgroups are dispatched round-robin over the 8 XCDs; renumber so each
  // XCD receives a contiguous range of tiles, then order tiles within a
  // plane in groups of kGroupM tile rows so that concurrently running tiles
  // share A and B panels in that XCD's L2.
  const uint32_t total = gridDim.x;
  uint32_t id = blockIdx.x;
  if ((total & 7u) == 0u) id = (id & 7u) * (total >> 3) + (id >> 3);
  const uint32_t tiles = tiles_m * tiles_n;
  const uint32_t pid = id % tiles;
  const uint32_t plane_slice = id / tiles;
  const uint32_t plane = plane_slice % args.nplanes;
  const uint32_t slice = plane_slice / args.nplanes;
  const uint32_t group = pid / (kGroupM * tiles_n);
  const uint32_t first_m = group * kGroupM;
  const uint32_t group_rows = min(tiles_m - first_m, static_cast<uint32_t>(kGroupM));
  const uint32_t tm = first_m + (pid % (kGroupM * tiles_n)) % group_rows;
  const uint32_t tn = (pid % (kGroupM * tiles_n)) / group_rows;

  const int8_t* const A = args.a + static_cast<int64_t>(plane) * args.pitch_a;
  const int8_t* const B = args.b + static_cast<int64_t>(plane) * args.pitch_b;
  const int64_t m0 = static_cast<int64_t>(tm) * kBM;
  const int64_t n0 = static_cast<int64_t>(tn) * kBN;
  const int64_t kbeg = k_begin + static_cast<int64_t>(slice) * k_slice;
  const int64_t kend = min(k_stop, kbeg + k_slice);
  const int ktiles = kend > kbeg ? static_cast<int>((kend - kbeg + BK - 1) / BK) : 0;

  // ---- global -> LDS by DMA ------------------------------------------------
  // buffer_load_dwordx4 ... lds writes lane l's 16 bytes to M0 + 16*l, so one
  // wave instruction fills a contiguous 1 KB block of a stage; each lane loads
  // the global bytes that belong in its slot (the LDS swizzle is applied on
  // the global side). Range checks come from the buffer resources and read
  // zero when out of range: A's covers the valid rows of this tile's row panel
  // from the current K offset on, B's the k rows [k0, min(k0 + BK, kend)).
  // B columns past the padded pitch get an offset beyond num_records.
  const int64_t a_rows = min(static_cast<int64_t>(kBM), args.m - m0);
  const int8_t* const a_panel = A + m0 * args.lda;
  uint32_t a_voff[T::kDma];  // wave w fills A rows 64w .. 64w+63 (4 blocks of 16 rows)
  uint32_t b_voff[T::kDma];  // wave w fills B k rows 16w .. 16w+15 (4 blocks of 4 rows)
#pragma unroll
  for (int i = 0; i < T::kDma; ++i) {
    const int blk = wave * T::kDma + i;
    const int row = 16 * blk + (lane >> 2);
    a_voff[i] = static_cast<uint32_t>(row * args.lda + 16 * swizzle_a(row, lane & 3));
    const int k = 4 * blk + (lane >> 4);
    const int64_t col = n0 + 16 * swizzle_b(k, lane & 15);
    b_voff[i] = static_cast<uint32_t>(k * args.ldb) + (col < args.ldb ? static_cast<uint32_t>(col) : 0x80000000u);
  }
  const uint32_t lds_base = lds_address(lds) + static_cast<uint32_t>(wave * T::kDma * 1024);

  struct TileSrc {
    v4i a, b;  // buffer resources of one K tile
  };
  auto tile_src = [&](int t) {
    const int64_t k0 = kbeg + static_cast<int64_t>(t) * BK;
    const int64_t a_bytes = a_rows * args.lda - k0;
    const int64_t rows_left = kend - k0;
    const int64_t b_rows = rows_left < BK ? (rows_left > 0 ? rows_left : 0) : BK;
    return TileSrc{buffer_rsrc(a_panel + k0, a_bytes > 0 ? a_bytes : 0), buffer_rsrc(B + k0 * args.ldb, b_rows * args.ldb)};
  };
  auto dma_a = [&](const TileSrc& src, int stage, int i) {
    dma16(lds_base + static_cast<uint32_t>(stage * T::kStage + 1024 * i), a_voff[i], src.a);
  };
  auto dma_b = [&](const TileSrc& src, int stage, int i) {
    dma16(lds_base + static_cast<uint32_t>(stage * T::kStage + T::kBufA + 1024 * i), b_voff[i], src.b);
  };
  auto issue_tile = [&](int t, int stage) {
    const TileSrc src = tile_src(t);
#pragma unroll
    for (int i = 0; i < T::kDma; ++i) dma_a(src, stage, i);
#pragma unroll
    for (int i = 0; i < T::kDma; ++i) dma_b(src, stage, i);
  };

  // ---- fragments -------------------------------------------------------------
  // K sub-step s covers k = 32s .. 32s+31 of a stage; lane l takes the 16 k
  // values 32s + 16*(l >> 5) + 0..15 for both operands.
  // A (MFMA src1): lane l holds row l & 31 of a 32-row block: one ds_read_b128.
  // B (MFMA src0): lane l holds column l & 31 of a 32-column block, gathered
  // by two ds_read_b64_tr_b8. In each 16-lane group, lane j addresses the
  // 8-byte row segment (k = base + (j >> 1), columns 8*(j & 1) .. +7 of the
  // group's 16 columns) and lane i receives byte i & 7 of the segments of
  // lanes 2b + (i >> 3), b = 0..7: its column across 8 consecutive k.
  const int frag_row = lane & 31;
  const int frag_half = lane >> 5;
  const int tr_j = lane & 15;
  const int tr_g = lane >> 4;
  struct Frags {
    v4i a[4];
    v4i b[4];
  };
  auto read_a = [&](int stage, int s, int i) {
    const int r = wave_m * 128 + 32 * i + frag_row;
    return *reinterpret_cast<const v4i*>(lds + stage * T::kStage + r * BK + swizzle_a(r, 2 * s + frag_half) * 16);
  };
  auto read_b = [&](int stage, int s, int j) {
    const int8_t* const sb = lds + stage * T::kStage + T::kBufA;
    const int ncol = wave_n * 128 + 32 * j + 16 * (tr_g & 1) + 8 * (tr_j & 1);
    const int k = 32 * s + 16 * (tr_g >> 1) + (tr_j >> 1);
    const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        as_lds_v2i(sb + k * kBN + swizzle_b(k, ncol >> 4) * 16 + (ncol & 8)));
    const v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        as_lds_v2i(sb + (k + 8) * kBN + swizzle_b(k + 8, ncol >> 4) * 16 + (ncol & 8)));
    return v4i{lo[0], lo[1], hi[0], hi[1]};
  };
  auto read_frags = [&](int stage, int s, Frags& f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f.a[i] = read_a(stage, s, i);
#pragma unroll
    for (int j = 0; j < 4; ++j) f.b[j] = read_b(stage, s, j);
  };

  v16i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v16i{} + kAccBias;

  auto mfma_rows = [&](const Frags& f, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[j], f.a[i], acc[i][j], 0, 0, 0);
  };

  // ---- pipeline ----------------------------------------------------------------
  // Four LDS stages. Step t computes tile t from stage t%4 while the DMA of
  // tile t+3 into stage (t+3)%4 (last read in step t-1) is in flight and the
  // first fragments of tile t+1 are prefetched. Before the barrier that ends
  // step t each wave waits until only its tile t+3 DMAs are outstanding, so
  // the barrier publishes tile t+2 (first read in step t+1) and retires every
  // read of stage t%4. Past the end of K the DMAs read zeros into stages no
  // later step reads, so the body has no branches. The DMAs are issued from
  // inline asm, so the compiler tracks no LDS write for them and adds no
  // waits before the fragment reads: the explicit vmcnt waits below are
  // what orders them.
  Frags f0, f1, f0n;
  issue_tile(0, 0);
  issue_tile(1, 1);
  issue_tile(2, 2);
  __builtin_amdgcn_s_waitcnt(kWaitVm[2 * T::kDma]);  // tiles 0 and 1 landed
  __syncthreads();
  read_frags(0, 0, f0);
  int stage = 0;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int stage1 = (stage + 1) & 3;
    const int stage3 = (stage + 3) & 3;
    // Region 1: sub-step 0 MFMAs; the sub-step 1 fragment reads with the A
    // DMAs of tile t+3 between them (source order fixes their placement).
    // The DMAs are spread over the whole step: each one occupies the texture
    // path for a while, and bunching all of a step's DMAs stalls MFMA issue.
    const TileSrc src = tile_src(kt + 3);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f1.a[i] = read_a(stage, 1, i);
      f1.b[i] = read_b(stage, 1, i);
      dma_a(src, stage3, i);
    }
    mfma_rows(f0, 0, 4);
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);  // DS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);
    __builtin_amdgcn_sched_barrier(0);
    // Region 2: sub-step 1 MFMAs; first fragments of tile t+1 with the B DMAs
    // of tile t+3 between them.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f0n.a[i] = read_a(stage1, 0, i);
      f0n.b[i] = read_b(stage1, 0, i);
      dma_b(src, stage3, i);
    }
    mfma_rows(f1, 0, 4);
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 2);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 2);  // DS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 2);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kWaitVm[2 * T::kDma]);  // only tile t+3 outstanding
    __syncthreads();
    f0 = f0n;
    stage = stage1;
  }
  __builtin_amdgcn_s_waitcnt(kWaitVm[0]);  // no DMA outlives the workgroup's LDS

  // ---- epilogue ---------------------------------------------------------------
  // acc[i][j] register 4g+e holds u = 2^31 + C[row][col] (mod 2^32; the
  // accumulators start at 2^31) with
  //   row = m0 + wave_m*128 + 32i + (lane & 31)
  //   col = n0 + wave_n*128 + 32j + 8g + 4*(lane >> 5) + e.
  // Stores go through a buffer resource over this tile's rows, so rows >= M
  // are dropped by the range check; columns past the padded pitch (only in
  // the last tile column) get an offset beyond num_records.
  const ModulusConsts mc = pc.mod[plane];
  const int64_t tile_rows = min(static_cast<int64_t>(kBM), args.m - m0);
  const uint32_t lane_off =
      static_cast<uint32_t>((wave_m * 128 + frag_row) * args.ldc + wave_n * 128 + 4 * frag_half);
  const uint32_t row_step = static_cast<uint32_t>(32 * args.ldc);
  const bool full_cols = n0 + kBN <= args.ldc;
  const int col_room = static_cast<int>(args.ldc - n0) - (wave_n * 128 + 4 * frag_half);
  auto col_off = [&](uint32_t off, int col) {  // col = 32j + 8g within the lane's wave tile
    return (full_cols || col < col_room) ? off + static_cast<uint32_t>(col) : 0x80000000u;
  };
  if (args.slices <= 1) {
    int8_t* const C = args.c + static_cast<int64_t>(plane) * args.pitch_c + m0 * args.ldc + n0;
    const __amdgpu_buffer_rsrc_t c_rsrc = make_rsrc(C, tile_rows * args.ldc - n0);
    const uint32_t m_comp = 256u - mc.m;
    const uint32_t half2 = mc.half * 0x00010001u;
    // The packed residues of each wave's 128 x 128 block go through LDS (free
    // once every wave's last DMA has landed) so the global stores are
    // row-contiguous 16-byte chunks: 8 full 128-byte lines per instruction.
    // LDS block layout: row-major, 128-byte rows, 16-byte chunk c of row r at
    // chunk position c ^ ((r >> 1) & 7) (2-way bank conflicts at most).
    __syncthreads();
    int8_t* const ep = lds + wave * (128 * 128);
    auto reduce = [&](auto carry) {
      constexpr bool kCarry = decltype(carry)::value;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t off = lane_off + static_cast<uint32_t>(i) * row_step;
        uint32_t prev[4][4];
        if constexpr (kCarry) {
          // later K block: add the centered residue carried in C (|.| <= 128)
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g)
              prev[j][g] = static_cast<uint32_t>(
                  __builtin_amdgcn_raw_buffer_load_b32(c_rsrc, static_cast<int>(off + 32 * j + 8 * g), 0, 0));
        }
        const int r = 32 * i + frag_row;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            uint32_t res[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              uint32_t u = static_cast<uint32_t>(acc[i][j][4 * g + e]);
              if constexpr (kCarry)
                u += static_cast<uint32_t>(static_cast<int32_t>(static_cast<int8_t>(prev[j][g] >> (8 * e))));
              res[e] = residue_plus_half(u, mc, m_comp);
            }
            const int c = 2 * j + (g >> 1);
            *reinterpret_cast<uint32_t*>(ep + r * 128 + ((c ^ ((r >> 1) & 7)) << 4) + 8 * (g & 1) +
                                         4 * frag_half) = pack_centered(res[0], res[1], res[2], res[3], half2);
          }
        }
      }
    };
    if (accumulate)
      reduce(std::true_type{});
    else
      reduce(std::false_type{});
    // Read back row-contiguous: lane l takes chunk l & 7 of rows 8q + (l >> 3).
    const int rrow = lane >> 3;
    const int rchunk = lane & 7;
    const bool chunk_ok = full_cols || wave_n * 128 + 16 * rchunk < static_cast<int>(args.ldc - n0);
    const uint32_t goff =
        static_cast<uint32_t>((wave_m * 128 + rrow) * args.ldc + wave_n * 128 + 16 * rchunk);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int row = 8 * q + rrow;
      const v4i v = *reinterpret_cast<const v4i*>(ep + row * 128 + ((rchunk ^ ((row >> 1) & 7)) << 4));
      const uint32_t o = goff + static_cast<uint32_t>(8 * q) * static_cast<uint32_t>(args.ldc);
      __builtin_amdgcn_raw_buffer_store_b128(v, c_rsrc, static_cast<int>(chunk_ok ? o : 0x80000000u), 0, 0);
    }
  } else {
    // Split-K: add this slice's partial sums (u - 2^31) into the int32
    // workspace [plane][M][ldc] with buffer atomics.
    int32_t* const W = args.splitk_ws + (static_cast<int64_t>(plane) * args.m + m0) * args.ldc + n0;
    const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(W, 4 * (tile_rows * args.ldc - n0));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t off = lane_off + static_cast<uint32_t>(i) * row_step;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t o = col_off(off, 32 * j + 8 * g);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            __builtin_amdgcn_raw_ptr_buffer_atomic_add_i32(acc[i][j][4 * g + e] ^ kAccBias, w_rsrc,
                                                       static_cast<int>(o == 0x80000000u ? o : 4 * (o + e)), 0, 0);
        }
    }
  }
}

// Reduce the summed split-K partials to int8 residues and clear the workspace.
// One thread per 4 consecutive cells of a plane row (ldc is a multiple of 16).
__global__ __launch_bounds__(256) void splitk_finalize_kernel(int32_t* ws, int8_t* c, int64_t m, int64_t ldc,
                                                              int64_t pitch_c, uint32_t nplanes, PlaneConsts pc,
                                                              uint32_t accumulate) {
  const int64_t words_per_plane = m * ldc / 4;
  const int64_t total = words_per_plane * nplanes;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; w < total;
       w += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const uint32_t plane = static_cast<uint32_t>(w / words_per_plane);
    const int64_t in_plane = w - static_cast<int64_t>(plane) * words_per_plane;
    const ModulusConsts mc = pc.mod[plane];
    v4i* const src = reinterpret_cast<v4i*>(ws + static_cast<int64_t>(plane) * m * ldc) + in_plane;
    const v4i v = *src;
    *src = v4i{0, 0, 0, 0};
    const int64_t elem = in_plane * 4;
    const int64_t row = elem / ldc;
    const int64_t col = elem - row * ldc;
    uint32_t* const dst = reinterpret_cast<uint32_t*>(c + static_cast<int64_t>(plane) * pitch_c + row * ldc + col);
    const uint32_t prev = accumulate ? *dst : 0u;
    uint32_t r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t u = (static_cast<uint32_t>(v[e]) ^ 0x80000000u) +
                         static_cast<uint32_t>(static_cast<int32_t>(static_cast<int8_t>(prev >> (8 * e))));
      r[e] = residue_plus_half(u, mc, 256u - mc.m);
    }
    *dst = pack_centered(r[0], r[1], r[2], r[3], mc.half * 0x00010001u);
  }
}

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* dst, uint64_t words) {
  for (uint64_t w = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; w < words;
       w += static_cast<uint64_t>(gridDim.x) * blockDim.x)
    dst[w] = 0u;
}

constexpr int kGemmBK = 64;
constexpr int64_t kSplitMaxLd = int64_t{1} << 21;

bool gemm_shape_ok(const GemmArgs& a) {
  if (a.m <= 0 || a.n <= 0 || a.k <= 0) return false;
  if (a.nplanes == 0 || a.nplanes > kMaxPrefix) return false;
  if (a.lda % 16 || a.ldb % 16 || a.ldc % 16) return false;
  if (a.lda < a.k || a.ldb < a.n || a.ldc < a.n) return false;
  // 32-bit buffer offsets: a 256-row panel and a BK-row slab must stay below 2^31
  if (a.lda >= (int64_t{1} << 23) || a.ldb >= (int64_t{1} << 23)) return false;
  if (a.ldc != a.ldb) return false;  // C columns == B columns: same padded pitch
  if (a.pitch_a < a.m * a.lda || a.pitch_b < a.k * a.ldb || a.pitch_c < a.m * a.ldc) return false;
  if (!a.a || !a.b || !a.c) return false;
  if (a.slices == 0) return false;
  if (a.slices > 1 && !a.splitk_ws) return false;
  // split-K workspace offsets are byte offsets of int32 cells in a 256-row tile
  if (a.slices > 1 && a.ldc >= kSplitMaxLd) return false;
  return true;
}

}  // namespace

uint32_t choose_splitk_slices(int64_t m, int64_t n, int64_t k, uint32_t nplanes) {
  // Enough workgroups to cover the 256 CUs at least twice; slices of at least
  // 2048 K so each slice still runs a long MFMA main loop.
  const int64_t tiles = ((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN) * static_cast<int64_t>(nplanes);
  const int64_t target = 512;
  if (tiles >= target / 2 || k < 4096 || padded_ld(n) >= kSplitMaxLd) return 1;
  int64_t slices = (target + tiles - 1) / tiles;
  const int64_t max_by_k = k / 2048;
  if (slices > max_by_k) slices = max_by_k;
  if (slices < 1) slices = 1;
  if (slices > 256) slices = 256;
  return static_cast<uint32_t>(slices);
}

uint64_t splitk_workspace_bytes(int64_t m, int64_t n, int64_t k, uint32_t nplanes) {
  if (choose_splitk_slices(m, n, k, nplanes) <= 1) return 0;
  const int64_t ldc = padded_ld(n);
  return static_cast<uint64_t>(nplanes) * static_cast<uint64_t>(m) * static_cast<uint64_t>(ldc) * 4u;
}

hipError_t launch_zero_words(uint32_t* dst, uint64_t words, hipStream_t stream) {
  if (words == 0) return hipSuccess;
  if (!dst) return hipErrorInvalidValue;
  const uint64_t blocks = (words + 255) / 256;
  const unsigned grid = static_cast<unsigned>(blocks < 4096 ? blocks : 4096);
  hipLaunchKernelGGL(zero_words_kernel, dim3(grid), dim3(256), 0, stream, dst, words);
  return hipGetLastError();
}

hipError_t launch_gemm(const GemmArgs& args, const PlaneConsts& consts, hipStream_t stream) {
  if (!gemm_shape_ok(args)) return hipErrorInvalidValue;
  const uint32_t tiles_m = static_cast<uint32_t>((args.m + kBM - 1) / kBM);
  const uint32_t tiles_n = static_cast<uint32_t>((args.ldc + kBN - 1) / kBN);
  const uint64_t words = static_cast<uint64_t>(args.nplanes) * args.m * args.ldc / 4;
  // K is processed in int32-safe blocks of 65536; a later block adds its sum
  // to the centered residue already in C (reference cpu_reference.cpp:160-175).
  for (int64_t kb = 0; kb < args.k; kb += kSafeKBlock) {
    const int64_t kstop = min(args.k, kb + kSafeKBlock);
    const uint32_t accumulate = kb > 0 ? 1u : 0u;
    int64_t k_slice = kstop - kb;
    uint32_t used_slices = 1;
    if (args.slices > 1) {
      k_slice = (k_slice + args.slices - 1) / args.slices;
      k_slice = (k_slice + kGemmBK - 1) / kGemmBK * kGemmBK;
      used_slices = static_cast<uint32_t>((kstop - kb + k_slice - 1) / k_slice);
    }
    const uint64_t blocks = static_cast<uint64_t>(tiles_m) * tiles_n * args.nplanes * used_slices;
    if (blocks == 0 || blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    hipLaunchKernelGGL(plane_gemm_kernel<kGemmBK>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, stream,
                       args, consts, tiles_m, tiles_n, kb, kstop, k_slice, accumulate);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (args.slices > 1) {
      const uint64_t fblocks = (words + 255) / 256;
      const unsigned grid = static_cast<unsigned>(fblocks < 8192 ? fblocks : 8192);
      hipLaunchKernelGGL(splitk_finalize_kernel, dim3(grid), dim3(256), 0, stream, args.splitk_ws, args.c, args.m,
                         args.ldc, args.pitch_c, args.nplanes, consts, accumulate);
      err = hipGetLastError();
      if (err != hipSuccess) return err;
    }
  }
  return hipSuccess;
}

}  // namespace rns8x
