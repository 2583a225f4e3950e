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
//   * K is consumed in BK-byte steps. A tile (256 x BK, K-contiguous rows) and
//     B tile (BK x 256, N-contiguous rows) are staged global -> VGPR -> LDS with
//     LDS double buffering: the global loads for step t+1 are issued before the
//     MFMAs of step t and written to the other LDS buffer after them, so one
//     barrier per step suffices.
//   * B arrives N-contiguous but the MFMA wants 16 K-contiguous bytes per lane,
//     so each thread loads BK/4 rows x 4 columns with dword loads (a wave reads
//     whole 256-byte rows, fully coalesced) and transposes 4x4 byte blocks with
//     v_perm_b32 before writing 16-byte K runs to LDS.
//   * LDS rows are BK bytes; 16-byte chunks are XOR-swizzled by row so that the
//     ds_read_b128 fragment loads of 8 (32-bank) or 16 (64-bank) consecutive
//     rows touch distinct banks.
//   * MFMA: v_mfma_i32_32x32x32_i8 with the B^T fragment as src0 and the A
//     fragment as src1, so each lane ends with 4 consecutive output columns
//     of one row per register group -> one packed dword store per group.
//   * Exactness: |a*b| <= 2^14, so <= 65536 products plus a carried residue
//     fit int32. Accumulators are reduced to centered residues in registers
//     every 65536 K and in the epilogue.
//   * Split-K (tall-skinny K): each slice reduces (when K > 65536) and
//     atomically adds its partial into an int32 workspace; a finalize kernel
//     reduces to int8 and clears the workspace.
#include "kernels.hpp"

namespace rns8x {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kThreads = 256;
constexpr int kGroupM = 4;  // tile rows per L2 reuse group
// Buffer resource word 3 for gfx9-family raw buffers (32-bit data format).
constexpr int kBufferFlags = 0x00020000;

template <int BK>
struct Tile {
  static constexpr int kChunks = BK / 16;                          // 16-byte chunks per LDS row
  static constexpr int kBufA = kBM * BK;                           // bytes per A buffer
  static constexpr int kBufB = kBN * BK;                           // bytes per B buffer
  static constexpr int kLds = 3 * (kBufA + kBufB);                 // 3-buffer ring
  static constexpr int kARowStep = kThreads / kChunks;             // rows covered per A load round
  static constexpr int kALoads = kBM * kChunks / kThreads;         // 16-byte A loads per thread
  static constexpr int kBRows = BK / 4;                            // B k-rows per wave (4 waves)
  static constexpr int kBGroups = kBRows / 16;                     // 16-row groups per wave
};

// XOR swizzle of the 16-byte chunk index by row bits 1-5. With BK = 64 (four
// chunks per row) it keeps every LDS access pattern of the kernel free of
// bank conflicts for both 32-bank/8-lane and 64-bank/16-lane ds_*_b128
// servicing: fragment reads (32 consecutive rows, one chunk), A staging writes
// (16 rows x 4 chunks) and the rotated B staging writes (rows 4*lane + (j +
// lane) % 4, one chunk); checked by an exhaustive model on the host.
template <int BK>
__device__ __forceinline__ int swizzle_chunk(int row, int chunk) {
  static_assert(BK == 64, "swizzle derived for 4 chunks per row");
  return chunk ^ (((row >> 1) & 3) ^ (((row >> 3) & 1) * 3) ^ ((row >> 4) & 3));
}

// Exact centered residue of an int32 (see tables.hpp): u = acc + 2^31 read as
// bytes, s = dot(bytes, 2^(8b) mod m) + (H - 2^31 mod m) < 2^18,
// q = umulhi(s, ceil(2^32/m)) = floor(s/m), result = s - q*m - H.
__device__ __forceinline__ int32_t reduce_centered(int32_t acc, uint32_t m, uint32_t half, uint32_t recip,
                                                   uint32_t pow_lo, uint32_t off) {
  const uint32_t u = static_cast<uint32_t>(acc) ^ 0x80000000u;
  const uint32_t s = __builtin_amdgcn_udot4(u, pow_lo, off, false);
  const uint32_t q = __umulhi(s, recip);
  return static_cast<int32_t>(s - q * m) - static_cast<int32_t>(half);
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

__device__ __forceinline__ uint32_t pack4(int32_t a, int32_t b, int32_t c, int32_t d) {
  return (static_cast<uint32_t>(a) & 0xFFu) | ((static_cast<uint32_t>(b) & 0xFFu) << 8) |
         ((static_cast<uint32_t>(c) & 0xFFu) << 16) | (static_cast<uint32_t>(d) << 24);
}

// 4x4 byte transpose: x_r holds bytes (row r, cols 0..3); y_c gets bytes
// (rows 0..3, col c). v_perm_b32(s0, s1, sel): selector 0-3 picks s1 bytes,
// 4-7 picks s0 bytes.
__device__ __forceinline__ void transpose4x4(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3, uint32_t& y0,
                                             uint32_t& y1, uint32_t& y2, uint32_t& y3) {
  const uint32_t t0 = __builtin_amdgcn_perm(x1, x0, 0x06020400u);  // x0.b0 x1.b0 x0.b2 x1.b2
  const uint32_t t1 = __builtin_amdgcn_perm(x1, x0, 0x07030501u);  // x0.b1 x1.b1 x0.b3 x1.b3
  const uint32_t t2 = __builtin_amdgcn_perm(x3, x2, 0x06020400u);
  const uint32_t t3 = __builtin_amdgcn_perm(x3, x2, 0x07030501u);
  y0 = __builtin_amdgcn_perm(t2, t0, 0x05040100u);  // t0.b0 t0.b1 t2.b0 t2.b1
  y2 = __builtin_amdgcn_perm(t2, t0, 0x07060302u);  // t0.b2 t0.b3 t2.b2 t2.b3
  y1 = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
  y3 = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

template <int BK>
__global__ __launch_bounds__(kThreads, 1) void plane_gemm_kernel(GemmArgs args, PlaneConsts pc, uint32_t tiles_m,
                                                                  uint32_t tiles_n, int64_t k_begin, int64_t k_stop,
                                                                  int64_t k_slice, uint32_t accumulate) {
  using T = Tile<BK>;
  static_assert(BK == 64, "fragment schedule below assumes two k32 sub-steps per K step");
  __shared__ __attribute__((aligned(16))) int8_t lds[T::kLds];

  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = tid >> 6;
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

  // ---- global -> register staging -----------------------------------------
  // Global loads go through raw buffer resources: every offset that needs a
  // range check is in the per-lane VGPR offset, which the hardware compares
  // with num_records and answers with zero when out of range. A's resource
  // covers the valid rows of this tile's row panel (rows >= M read as zero);
  // B's resource is rebuilt per K step to cover only rows [k0, min(k0+BK,
  // kend)), so rows past the slice or past K read as zero. Columns past the
  // padded pitch get an offset beyond num_records.
  const int a_chunk = tid % T::kChunks;
  const int a_row0 = tid / T::kChunks;
  v4i a_stage[T::kALoads];
  uint32_t b_stage[T::kBRows];
  const int64_t a_rows = min(static_cast<int64_t>(kBM), args.m - m0);
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(A + m0 * args.lda, a_rows * args.lda);
  const uint32_t a_voff = static_cast<uint32_t>(a_row0 * args.lda + 16 * a_chunk);
  const int64_t b_col = n0 + 4 * lane;
  const uint32_t b_voff = static_cast<uint32_t>(wave * T::kBRows * args.ldb) +
                          (b_col < args.ldb ? static_cast<uint32_t>(b_col) : 0x80000000u);

  auto load_a = [&](int t) {
    const int64_t k0 = kbeg + static_cast<int64_t>(t) * BK;
#pragma unroll
    for (int i = 0; i < T::kALoads; ++i) {
      const uint32_t uni = static_cast<uint32_t>(k0 + static_cast<int64_t>(i) * T::kARowStep * args.lda);
      a_stage[i] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, static_cast<int>(a_voff + uni), 0, 0);
    }
  };
  auto load_b = [&](int t) {
    const int64_t k0 = kbeg + static_cast<int64_t>(t) * BK;
    const int64_t rows_left = kend - k0;
    const int64_t b_rows = rows_left < BK ? (rows_left > 0 ? rows_left : 0) : BK;
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(B + k0 * args.ldb, b_rows * args.ldb);
#pragma unroll
    for (int i = 0; i < T::kBRows; ++i) {
      const uint32_t uni = static_cast<uint32_t>(i * args.ldb);
      b_stage[i] =
          static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(b_rsrc, static_cast<int>(b_voff + uni), 0, 0));
    }
  };
  auto load_tile = [&](int t) {
    load_a(t);
    load_b(t);
  };

  // ---- register -> LDS (3-buffer ring; B transposed to K-contiguous rows) --
  auto store_a = [&](int buf) {
    int8_t* const la = lds + buf * (T::kBufA + T::kBufB);
#pragma unroll
    for (int i = 0; i < T::kALoads; ++i) {
      const int r = a_row0 + i * T::kARowStep;
      *reinterpret_cast<v4i*>(la + r * BK + swizzle_chunk<BK>(r, a_chunk) * 16) = a_stage[i];
    }
  };
  auto store_b = [&](int buf) {
    int8_t* const lb = lds + buf * (T::kBufA + T::kBufB) + T::kBufA;
    // Each lane holds a 16-row x 4-column byte block of B. The block is
    // transposed to 4 columns x 16 K bytes; the 4 output columns are emitted in
    // an order rotated by (lane & 3) so the rows one write instruction touches
    // cover all residues mod 4 (rows 4*lane + (j + lane) % 4), which keeps the
    // writes bank-conflict free. The rotation is a per-lane byte rotate of each
    // input dword before the fixed 4x4 transpose.
    const uint32_t rot = static_cast<uint32_t>(lane & 3);
#pragma unroll
    for (int g = 0; g < T::kBGroups; ++g) {
      uint32_t y[4][4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int base = 16 * g + 4 * q;
        const uint32_t x0 = __builtin_amdgcn_alignbyte(b_stage[base], b_stage[base], rot);
        const uint32_t x1 = __builtin_amdgcn_alignbyte(b_stage[base + 1], b_stage[base + 1], rot);
        const uint32_t x2 = __builtin_amdgcn_alignbyte(b_stage[base + 2], b_stage[base + 2], rot);
        const uint32_t x3 = __builtin_amdgcn_alignbyte(b_stage[base + 3], b_stage[base + 3], rot);
        transpose4x4(x0, x1, x2, x3, y[q][0], y[q][1], y[q][2], y[q][3]);
      }
      const int chunk = (wave * T::kBRows) / 16 + g;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * lane + ((j + static_cast<int>(rot)) & 3);
        const v4i v = {static_cast<int>(y[0][j]), static_cast<int>(y[1][j]), static_cast<int>(y[2][j]),
                       static_cast<int>(y[3][j])};
        *reinterpret_cast<v4i*>(lb + r * BK + swizzle_chunk<BK>(r, chunk) * 16) = v;
      }
    }
  };
  auto store_tile = [&](int buf) {
    store_a(buf);
    store_b(buf);
  };

  // ---- fragments -------------------------------------------------------------
  const int frag_row = lane & 31;
  const int frag_half = lane >> 5;
  struct Frags {
    v4i a[4];
    v4i b[4];
  };
  auto read_frags = [&](int buf, int s, Frags& f) {
    const int8_t* const la = lds + buf * (T::kBufA + T::kBufB);
    const int8_t* const lb = la + T::kBufA;
    const int c = 2 * s + frag_half;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = wave_m * 128 + 32 * i + frag_row;
      f.a[i] = *reinterpret_cast<const v4i*>(la + r * BK + swizzle_chunk<BK>(r, c) * 16);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = wave_n * 128 + 32 * j + frag_row;
      f.b[j] = *reinterpret_cast<const v4i*>(lb + r * BK + swizzle_chunk<BK>(r, c) * 16);
    }
  };

  v16i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v16i{};

  auto mfma_rows = [&](const Frags& f, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[j], f.a[i], acc[i][j], 0, 0, 0);
  };

  // ---- pipeline ----------------------------------------------------------------
  // Three LDS ring buffers. Step t computes tile t from buffer t%3 while
  //   * tile t+2 (loaded into registers during step t-1) is transposed and
  //     written to buffer (t+2)%3, last read in step t-1;
  //   * the global loads of tile t+3 are issued (consumed in step t+1, so a
  //     whole step hides their latency);
  //   * the first fragments of tile t+1 are prefetched from buffer (t+1)%3,
  //     complete since the barrier that ended step t-1.
  // The barrier ending step t publishes tile t+2 and retires all reads of
  // buffer t%3. Past the end of K the loads return zeros and land in buffers
  // no later step reads, so the body has no branches and is one scheduling
  // region.
  Frags f0, f1, f0n;
  load_tile(0);
  store_tile(0);
  load_tile(1);
  store_tile(1);
  load_tile(2);
  __syncthreads();
  read_frags(0, 0, f0);
  int buf = 0;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int buf1 = buf == 2 ? 0 : buf + 1;
    const int buf2 = buf1 == 2 ? 0 : buf1 + 1;
    // Region 1: sub-step-1 fragment reads issued first (consumed in region 3),
    // half of the sub-step-0 MFMAs, A staging store + next A loads.
    read_frags(buf, 1, f1);
    mfma_rows(f0, 0, 2);
    store_a(buf2);
    load_a(kt + 3);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x080, 2, 1);  // DS
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 1);  // VMEM read
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 1);  // VALU
    }
    __builtin_amdgcn_sched_barrier(0);
    // Region 2: rest of sub-step 0; B transpose + store + next B loads.
    mfma_rows(f0, 2, 4);
    store_b(buf2);
    load_b(kt + 3);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 2);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 8, 2);  // VALU (rotate, transpose, offsets)
      __builtin_amdgcn_sched_group_barrier(0x080, 1, 2);  // DS write
      __builtin_amdgcn_sched_group_barrier(0x020, 2, 2);  // VMEM read
    }
    __builtin_amdgcn_sched_barrier(0);
    // Region 3: sub-step 1; prefetch of the next tile's first fragments.
    read_frags(buf1, 0, f0n);
    mfma_rows(f1, 0, 4);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 3);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 3);  // DS read
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    f0 = f0n;
    buf = buf1;
  }

  // ---- epilogue ---------------------------------------------------------------
  // acc[i][j] register 4g+e holds C[row][col] with
  //   row = m0 + wave_m*128 + 32i + (lane & 31)
  //   col = n0 + wave_n*128 + 32j + 8g + 4*(lane >> 5) + e
  const ModulusConsts mc = pc.mod[plane];
  if (args.slices <= 1) {
    int8_t* const C = args.c + static_cast<int64_t>(plane) * args.pitch_c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = m0 + wave_m * 128 + 32 * i + frag_row;
      const bool row_ok = row < args.m;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t col = n0 + wave_n * 128 + 32 * j + 8 * g + 4 * frag_half;
          const bool ok = row_ok && col < args.ldc;
          uint32_t* const dst = reinterpret_cast<uint32_t*>(C + row * args.ldc + col);
          int32_t v0 = acc[i][j][4 * g + 0], v1 = acc[i][j][4 * g + 1];
          int32_t v2 = acc[i][j][4 * g + 2], v3 = acc[i][j][4 * g + 3];
          if (accumulate && ok) {
            // later K block: add the centered residue carried in C (|.| <= 128)
            const uint32_t prev = *dst;
            v0 += static_cast<int8_t>(prev);
            v1 += static_cast<int8_t>(prev >> 8);
            v2 += static_cast<int8_t>(prev >> 16);
            v3 += static_cast<int8_t>(prev >> 24);
          }
          const int32_t r0 = reduce_centered(v0, mc.m, mc.half, mc.recip, mc.pow_lo, mc.off_i32);
          const int32_t r1 = reduce_centered(v1, mc.m, mc.half, mc.recip, mc.pow_lo, mc.off_i32);
          const int32_t r2 = reduce_centered(v2, mc.m, mc.half, mc.recip, mc.pow_lo, mc.off_i32);
          const int32_t r3 = reduce_centered(v3, mc.m, mc.half, mc.recip, mc.pow_lo, mc.off_i32);
          if (ok) *dst = pack4(r0, r1, r2, r3);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  } else {
    int32_t* const W = args.splitk_ws + static_cast<int64_t>(plane) * args.m * args.ldc;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = m0 + wave_m * 128 + 32 * i + frag_row;
      const bool row_ok = row < args.m;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t col = n0 + wave_n * 128 + 32 * j + 8 * g + 4 * frag_half;
          if (row_ok && col < args.ldc) {
#pragma unroll
            for (int e = 0; e < 4; ++e) atomicAdd(W + row * args.ldc + col + e, acc[i][j][4 * g + e]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

// Reduce the summed split-K partials to int8 residues and clear the workspace.
__global__ __launch_bounds__(256) void splitk_finalize_kernel(int32_t* ws, int8_t* c, int64_t m, int64_t ldc,
                                                              int64_t pitch_c, uint32_t nplanes, PlaneConsts pc,
                                                              uint32_t accumulate) {
  const int64_t words_per_plane = m * ldc / 4;  // ldc is a multiple of 16
  const int64_t total = words_per_plane * nplanes;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; w < total;
       w += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const uint32_t plane = static_cast<uint32_t>(w / words_per_plane);
    const int64_t in_plane = w - static_cast<int64_t>(plane) * words_per_plane;
    const ModulusConsts mc = pc.mod[plane];
    v4i* const src = reinterpret_cast<v4i*>(ws + static_cast<int64_t>(plane) * m * ldc) + in_plane;
    v4i v = *src;
    *src = v4i{0, 0, 0, 0};
    const int64_t elem = in_plane * 4;
    const int64_t row = elem / ldc;
    const int64_t col = elem - row * ldc;
    uint32_t* const dst = reinterpret_cast<uint32_t*>(c + static_cast<int64_t>(plane) * pitch_c + row * ldc + col);
    if (accumulate) {
      const uint32_t prev = *dst;
      v[0] += static_cast<int8_t>(prev);
      v[1] += static_cast<int8_t>(prev >> 8);
      v[2] += static_cast<int8_t>(prev >> 16);
      v[3] += static_cast<int8_t>(prev >> 24);
    }
    const int32_t r0 = reduce_centered(v[0], mc.m, mc.half, mc.recip, mc.pow_lo, mc.off_i32);
    const int32_t r1 = reduce_centered(v[1], mc.m, mc.half, mc.recip, mc.pow_lo, mc.off_i32);
    const int32_t r2 = reduce_centered(v[2], mc.m, mc.half, mc.recip, mc.pow_lo, mc.off_i32);
    const int32_t r3 = reduce_centered(v[3], mc.m, mc.half, mc.recip, mc.pow_lo, mc.off_i32);
    *dst = pack4(r0, r1, r2, r3);
  }
}

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* dst, uint64_t words) {
  for (uint64_t w = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; w < words;
       w += static_cast<uint64_t>(gridDim.x) * blockDim.x)
    dst[w] = 0u;
}

constexpr int kGemmBK = 64;

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
  return true;
}

}  // namespace

uint32_t choose_splitk_slices(int64_t m, int64_t n, int64_t k, uint32_t nplanes) {
  // Enough workgroups to cover the 256 CUs at least twice; slices of at least
  // 2048 K so each slice still runs a long MFMA main loop.
  const int64_t tiles = ((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN) * static_cast<int64_t>(nplanes);
  const int64_t target = 512;
  if (tiles >= target / 2 || k < 4096) return 1;
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
