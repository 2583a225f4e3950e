// Plane-batched int8 MFMA GEMM for gfx950 (CDNA4).
//
// One launch computes C_p = center(A_p x B_p mod m_p) for every residue plane
// p (reference semantics: src/cpu/cpu_reference.cpp:156-206, the per-modulus
// ring GEMM with int32 accumulation reduced at least every 65536 K).
//
// Work decomposition
//   * unit = one output tile of one plane (and one K slice when split-K is
//     on). A persistent grid of workgroups (one per resident slot, a
//     multiple of 8) walks the unit list, each XCD a contiguous share, so the
//     DMA stream runs on across unit boundaries.
//   * workgroup = 256 threads (4 wave64s); waves form a 2x2 grid over the
//     tile. Two tile configurations: 256x256 (128x128 per wave, 16 MFMA
//     accumulators, one workgroup per CU) for large outputs and 128x128
//     (64x64 per wave, two workgroups per CU) when 256x256 tiles would leave
//     CUs idle.
//   * K is consumed in BK = 64 byte steps through a 4-stage LDS ring. Both
//     operands go global -> LDS by buffer-load DMA (no VGPR staging): A tiles
//     (BM x 64, K-contiguous rows) and B tiles (64 x BN, N-contiguous rows,
//     the layout they have in HBM). The DMA three K steps ahead is in flight
//     while a step computes, also across the epilogue into the next unit;
//     one barrier per step.
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
//     reciprocal quotient (full-rate VALU only); 4 residues are packed per
//     dword and staged through a per-wave LDS region (outside the stage
//     ring) into row-contiguous 16-byte stores.
//   * Split-K (few output tiles, 128x128 tiles): one launch covers the
//     whole K; each slice (at most 65536 K) reduces its tile like an
//     unsplit unit and stores the centered residues to its own slot of an
//     int8 workspace; residue_finalize adds the slots and writes C
//     (deterministic, no atomics, a quarter of the bytes int32 partials
//     would move).
//   * Results at most 16 columns wide run in skinny.hip instead.
#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "dma.hpp"
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
constexpr int kWaitVm[9] = {wait_vm(0), wait_vm(1), wait_vm(2), wait_vm(3), wait_vm(4),
                            wait_vm(5), wait_vm(6), wait_vm(7), wait_vm(8)};

constexpr int kThreads = 256;
constexpr int kGroupM = 4;  // tile rows per L2 reuse group
// Accumulator start value: the MFMAs then produce u = 2^31 + sum (mod 2^32),
// the biased form the reduction reads (|sum| < 2^31).
constexpr int kAccBias = static_cast<int>(0x80000000u);

// Tile configuration: each of the 4 waves (a 2 x 2 grid) owns WM x WN blocks
// of 32 x 32 outputs, so a workgroup tile is (64 WM) x (64 WN). K steps are 64
// bytes through 4 LDS stages.
template <int WM, int WN>
struct Cfg {
  static constexpr int kWM = WM, kWN = WN;
  static constexpr int BM = 64 * WM, BN = 64 * WN, BK = 64;
  static constexpr int kBufA = BM * BK;               // A stage: BM rows x 64 bytes
  static constexpr int kBufB = BK * BN;               // B stage: 64 k-rows x BN bytes
  static constexpr int kStage = kBufA + kBufB;
  static constexpr int kStages = 4;
  static constexpr int kLds = kStages * kStage;
  static constexpr int kDmaA = kBufA / 4096;          // 1 KB DMA blocks per wave (4 waves)
  static constexpr int kDmaB = kBufB / 4096;
  static constexpr int kChunksB = BN / 16;            // 16-byte chunks per B stage row
  static constexpr int kRowsPerBlockB = 1024 / BN;    // k rows per 1 KB B block
  static constexpr int kEpiRow = 32 * WN;             // bytes of one wave's output row
  static constexpr int kEpiChunks = kEpiRow / 16;
  static constexpr int kEpiRowsPerStore = 64 / kEpiChunks;
  static constexpr int kEpiBytes = 32 * WM * kEpiRow; // one wave's output block
  // The epilogue stages output through its own LDS region after the stage
  // ring, in kEpiParts passes (two for 256x256 tiles: 4 waves x 8 KB).
  static constexpr int kEpiParts = WM >= 4 ? 2 : 1;
  static constexpr int kEpiLds = 4 * kEpiBytes / kEpiParts;
  static_assert(kDmaA >= 1 && kDmaB >= 1 && WM % kEpiParts == 0, "tile config");
  static_assert(kLds + kEpiLds <= 160 * 1024, "LDS per workgroup");
};

// A stage: row-major BM x 64 bytes. The 16-byte chunk index is XORed with row
// bits 1-5 so the ds_read_b128 fragment loads (32 consecutive rows, one chunk)
// are bank-conflict free for both 32-bank/8-lane and 64-bank/16-lane
// servicing (exhaustive host model).
__device__ __forceinline__ int swizzle_a(int row, int chunk) {
  return chunk ^ (((row >> 1) & 3) ^ (((row >> 3) & 1) * 3) ^ ((row >> 4) & 3));
}

// B stage: row-major 64 (k) x BN bytes, N-contiguous as in global memory. A
// 16-lane transpose read touches 8 consecutive k rows of one chunk; the chunk
// index is XORed with f(k & 7) so those rows (and, in the 64-bank model, the
// neighbouring group's) land in distinct bank quads: f(x) = 2x mod 16 + x / 4
// for 16-chunk rows, f(x) = x for 8-chunk rows (exhaustive host model).
template <int BN>
__device__ __forceinline__ int swizzle_b(int k, int chunk) {
  const int x = k & 7;
  if constexpr (BN == 256)
    return chunk ^ (((2 * x) & 15) | (x >> 2));
  else
    return chunk ^ x;
}


// Scheduling slots of a K sub-step region: slot Q is one MFMA followed by up
// to kPerSlot of the region's kReads LDS fragment reads.
template <int kId, int Q, int kSlots, int kPerSlot, int kReads>
__device__ __forceinline__ void sched_slots() {
  if constexpr (Q < kSlots) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, kId);  // MFMA
    constexpr int kLeft = kReads - Q * kPerSlot;
    constexpr int kNum = kLeft < kPerSlot ? kLeft : kPerSlot;
    if constexpr (kNum > 0) __builtin_amdgcn_sched_group_barrier(0x100, kNum, kId);  // DS read
    sched_slots<kId, Q + 1, kSlots, kPerSlot, kReads>();
  }
}

// Work list of one launch: units (K slice, plane, output tile) are numbered
// slice-major, then plane, then tile; tiles run in groups of kGroupM tile
// rows. The divisors carry host-computed reciprocals (make_div_u31).
struct UnitMap {
  uint32_t units;
  uint32_t tiles_m;
  DivU31 tiles;   // tiles per plane
  DivU31 planes;  // planes
  DivU31 group;   // kGroupM * tiles_n: tiles per group of tile rows
  DivU31 rows;    // kGroupM: tile rows of a full group
  DivU31 tail;    // tile rows of the last group (tiles_m - its first row)
  uint32_t k_begin, k_stop, k_slice;
  // listed launches: two words per unit, (plane << 24 | tile row) and
  // (quadrant mask << 24 | tile column), in place of the arithmetic order
  const uint32_t* list;
  // grouped launches: units are numbered task-major, task_units per task
  DivU31 task_units;
};

// Grouped launches carry their tasks' base pointers by value (kernel
// arguments are read through the scalar cache); other launches an empty
// struct.
struct TaskTable {
  TaskPtrs t[kMaxGroupTasks];
};
struct NoTaskTable {};
template <bool kGrouped>
using GroupArg = std::conditional_t<kGrouped, TaskTable, NoTaskTable>;

// floor(n / d) for n < 2^31 (make_div_u31).
__device__ __forceinline__ uint32_t div_u31(uint32_t n, DivU31 v) { return __umulhi(n << 1, v.mul) >> v.shift; }

template <typename C, int kMinBlocks, bool kUniform, bool kListed = false, bool kGrouped = false>
__global__ __launch_bounds__(kThreads, kMinBlocks) void plane_gemm_kernel(GemmArgs args, PlaneConsts pc, UnitMap map,
                                                                           uint32_t accumulate,
                                                                           GroupArg<kGrouped> tasks) {
  constexpr int WM = C::kWM, WN = C::kWN, BM = C::BM, BN = C::BN, BK = C::BK;
  __shared__ __attribute__((aligned(16))) int8_t lds[C::kLds + C::kEpiLds];

  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wave_m = wave >> 1;
  const int wave_n = wave & 1;

  // ---- persistent work list ----------------------------------------------------
  // A unit is one (K slice, plane, output tile). The grid holds a few
  // workgroups per CU and each walks its units in order, so the DMA stream
  // runs on across unit boundaries: the next unit's first K tiles land while
  // the current unit's epilogue runs. Workgroups are dispatched round-robin
  // over the 8 XCDs; with a grid that is a multiple of 8, XCD x owns the
  // contiguous unit range [x*units/8, (x+1)*units/8), walked by its
  // workgroups in lock step, so concurrently running tiles are neighbours and
  // share A and B panels in that XCD's L2 (tiles are ordered within a plane
  // in groups of kGroupM tile rows).
  const uint32_t grid = gridDim.x;
  uint32_t u_first, u_step, u_end;
  if ((grid & 7u) == 0u) {
    const uint32_t xcd = blockIdx.x & 7u;
    u_first = static_cast<uint32_t>((static_cast<uint64_t>(xcd) * map.units) / 8) + (blockIdx.x >> 3);
    u_end = static_cast<uint32_t>((static_cast<uint64_t>(xcd + 1) * map.units) / 8);
    u_step = grid >> 3;
  } else {
    u_first = blockIdx.x;
    u_end = map.units;
    u_step = grid;
  }
  u_first = __builtin_amdgcn_readfirstlane(u_first);
  u_end = __builtin_amdgcn_readfirstlane(u_end);

  // Units are decoded on the scalar unit (every value here is uniform) with
  // the host's reciprocals, branch-free, so the cursor below can advance
  // every K step without splitting the loop body.
  struct Unit {
    uint32_t task, plane, slice, m0, n0, kbeg, kend, ktiles, quad;
  };
  // Listed units come from a per-tile schedule: a BM x BN tile of one plane
  // whose four quadrants (one per wave, 2 x 2) are stored only where the mask
  // has their bit (wave_m * 2 + wave_n); quadrants outside the tiles that
  // select this plane keep their contents.
  static_assert(kThreads == 256, "quadrant masks assume four waves in a 2 x 2 grid");
  auto decode = [&](uint32_t u) {
    Unit U;
    U.task = 0;
    if constexpr (kGrouped) {
      U.task = div_u31(u, map.task_units);
      u -= U.task * map.task_units.d;
    }
    if constexpr (kListed) {
      const uint32_t w0 = map.list[2u * u], w1 = map.list[2u * u + 1u];
      U.plane = w0 >> 24;
      U.slice = 0;
      U.m0 = (w0 & 0xFFFFFFu) * BM;
      U.n0 = (w1 & 0xFFFFFFu) * BN;
      U.quad = w1 >> 24;
      U.kbeg = map.k_begin;
      U.kend = map.k_stop;
      U.ktiles = (U.kend - U.kbeg + BK - 1) / BK;
      return U;
    }
    U.quad = 0xFu;
    const uint32_t plane_slice = div_u31(u, map.tiles);
    const uint32_t pid = u - plane_slice * map.tiles.d;
    U.slice = div_u31(plane_slice, map.planes);
    U.plane = plane_slice - U.slice * map.planes.d;
    const uint32_t group = div_u31(pid, map.group);
    const uint32_t first_m = group * kGroupM;
    const uint32_t rem = pid - group * map.group.d;
    const DivU31 rows = first_m + kGroupM <= map.tiles_m ? map.rows : map.tail;
    const uint32_t tn = div_u31(rem, rows);
    U.m0 = (first_m + rem - tn * rows.d) * BM;
    U.n0 = tn * BN;
    U.kbeg = map.k_begin + U.slice * map.k_slice;
    U.kend = min(map.k_stop, U.kbeg + map.k_slice);
    U.ktiles = U.kend > U.kbeg ? (U.kend - U.kbeg + BK - 1) / BK : 0u;
    return U;
  };

  // Base pointers of a unit's task (the launch's own in ungrouped launches).
  auto base_a = [&](const Unit& U) -> const int8_t* {
    if constexpr (kGrouped) return tasks.t[U.task].a;
    else return args.a;
  };
  auto base_b = [&](const Unit& U) -> const int8_t* {
    if constexpr (kGrouped) return tasks.t[U.task].b;
    else return args.b;
  };
  auto base_c = [&](const Unit& U) -> int8_t* {
    if constexpr (kGrouped) return tasks.t[U.task].c;
    else return args.c;
  };
  auto base_ws = [&](const Unit& U) -> int8_t* {
    if constexpr (kGrouped) return tasks.t[U.task].ws;
    else return args.splitk_ws;
  };

  // ---- global -> LDS by DMA ------------------------------------------------
  // buffer_load_dwordx4 ... lds writes lane l's 16 bytes to M0 + 16*l, so one
  // wave instruction fills a contiguous 1 KB block of a stage; each lane loads
  // the global bytes that belong in its slot (the LDS swizzle is applied on
  // the global side). The lane offsets are fixed; the K tile moves the
  // buffer resources. Range checks come from the resources and read zero when
  // out of range: A's covers the valid rows of the unit's row panel from the
  // current K offset on, B's the k rows [k0, min(k0 + BK, kend)) from column
  // n0 on. B columns past the padded pitch read the next k row (zero past the
  // resource): they only feed output columns >= ldc, which are never stored.
  const uint32_t lda = static_cast<uint32_t>(args.lda), ldb = static_cast<uint32_t>(args.ldb);
  const uint32_t m_rows = static_cast<uint32_t>(args.m);
  uint32_t a_voff[C::kDmaA];  // wave w fills A rows [16 kDmaA w, 16 kDmaA (w + 1))
  uint32_t b_voff[C::kDmaB];  // wave w fills B k rows [kRowsPerBlockB kDmaB w, ...)
#pragma unroll
  for (int i = 0; i < C::kDmaA; ++i) {
    const int row = 16 * (wave * C::kDmaA + i) + (lane >> 2);
    a_voff[i] = static_cast<uint32_t>(row) * lda + static_cast<uint32_t>(16 * swizzle_a(row, lane & 3));
  }
#pragma unroll
  for (int i = 0; i < C::kDmaB; ++i) {
    const int k = C::kRowsPerBlockB * (wave * C::kDmaB + i) + lane / C::kChunksB;
    b_voff[i] = static_cast<uint32_t>(k) * ldb + static_cast<uint32_t>(16 * swizzle_b<BN>(k, lane % C::kChunksB));
  }
  const uint32_t lds_a = lds_address(lds) + static_cast<uint32_t>(wave * C::kDmaA * 1024);
  const uint32_t lds_b = lds_address(lds) + static_cast<uint32_t>(C::kBufA + wave * C::kDmaB * 1024);

  // DMA cursor: the (unit, K tile) whose DMA is issued next, three K tiles
  // ahead of the compute position, and nsrc, its buffer resources. Past the
  // last unit the resources are empty (every lane reads zero), which keeps
  // the per-step DMA count and therefore the vmcnt bookkeeping uniform.
  struct TileSrc {
    v4i a, b;
  };
  uint32_t du = u_first, dkt = 0;
  Unit dU = decode(u_first);
  TileSrc nsrc;
  auto cursor_load = [&]() {
    const bool live = du < u_end;
    const uint32_t k0 = dU.kbeg + dkt * BK;
    const uint32_t a_rows = min(static_cast<uint32_t>(BM), m_rows - dU.m0);
    const uint32_t b_rows = min(static_cast<uint32_t>(BK), dU.kend - k0);
    const int8_t* const a_panel = base_a(dU) + static_cast<uint64_t>(dU.plane) * args.pitch_a +
                                  static_cast<uint64_t>(dU.m0) * lda;
    const int8_t* const b_slab = base_b(dU) + static_cast<uint64_t>(dU.plane) * args.pitch_b +
                                 static_cast<uint64_t>(k0) * ldb + dU.n0;
    nsrc = TileSrc{buffer_rsrc(a_panel + k0, live ? a_rows * lda - k0 : 0u),
                   buffer_rsrc(b_slab, live ? b_rows * ldb - dU.n0 : 0u)};
  };
  // General advance: decodes the cursor's unit at every step (the prologue,
  // and launches whose units differ in K tiles). With uniform units
  // (kUniform) the cursor crosses exactly one unit boundary per compute unit
  // (it advances one unit's K tiles per unit), so the unit after the
  // cursor's is decoded once per compute unit (next_du) and the per-step
  // advance is only selects: decoding at every step cost ~4% of the kernel.
  Unit nU = dU;
  auto cursor_advance = [&](auto uniform) {
    constexpr bool kFast = decltype(uniform)::value;
    const bool next_unit = dkt + 1 >= dU.ktiles;
    du = next_unit ? min(du + u_step, u_end) : du;
    dkt = next_unit ? 0u : dkt + 1;
    if constexpr (!kFast) nU = decode(min(du, u_end - 1));
    if (next_unit) dU = nU;
    cursor_load();
  };
  // (past the last unit any decoded unit will do: the resources are empty)
  auto next_du = [&]() { nU = decode(min(du + u_step, u_end - 1)); };
  cursor_load();
  auto dma_a = [&](const TileSrc& src, int stage, int i) {
    dma16(lds_a + static_cast<uint32_t>(stage * C::kStage + 1024 * i), a_voff[i], src.a);
  };
  auto dma_b = [&](const TileSrc& src, int stage, int i) {
    dma16(lds_b + static_cast<uint32_t>(stage * C::kStage + 1024 * i), b_voff[i], src.b);
  };
  auto issue_next = [&](int stage) {
#pragma unroll
    for (int i = 0; i < C::kDmaA; ++i) dma_a(nsrc, stage, i);
#pragma unroll
    for (int i = 0; i < C::kDmaB; ++i) dma_b(nsrc, stage, i);
    cursor_advance(std::false_type{});
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
    v4i a[WM];
    v4i b[WN];
  };
  auto read_a = [&](int stage, int s, int i) {
    const int r = wave_m * (32 * WM) + 32 * i + frag_row;
    return *reinterpret_cast<const v4i*>(lds + stage * C::kStage + r * BK + swizzle_a(r, 2 * s + frag_half) * 16);
  };
  auto read_b = [&](int stage, int s, int j) {
    const int8_t* const sb = lds + stage * C::kStage + C::kBufA;
    const int ncol = wave_n * (32 * WN) + 32 * j + 16 * (tr_g & 1) + 8 * (tr_j & 1);
    const int k = 32 * s + 16 * (tr_g >> 1) + (tr_j >> 1);
    const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        as_lds_v2i(sb + k * BN + swizzle_b<BN>(k, ncol >> 4) * 16 + (ncol & 8)));
    const v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        as_lds_v2i(sb + (k + 8) * BN + swizzle_b<BN>(k + 8, ncol >> 4) * 16 + (ncol & 8)));
    return v4i{lo[0], lo[1], hi[0], hi[1]};
  };
  auto read_frags = [&](int stage, int s, Frags& f) {
#pragma unroll
    for (int i = 0; i < WM; ++i) f.a[i] = read_a(stage, s, i);
#pragma unroll
    for (int j = 0; j < WN; ++j) f.b[j] = read_b(stage, s, j);
  };

  v16i acc[WM][WN];
  auto reset_acc = [&]() {
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j) acc[i][j] = v16i{} + kAccBias;
  };
  auto mfma_all = [&](const Frags& f) {
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[j], f.a[i], acc[i][j], 0, 0, 0);
  };
  // Interleave a region's WM*WN MFMAs with its WM + 2*WN fragment reads: the
  // reads go between the first three quarters of the MFMAs.
  constexpr int kMfma = WM * WN;
  constexpr int kReads = WM + 2 * WN;
  constexpr int kSlots = kMfma - kMfma / 4;
  constexpr int kPerSlot = (kReads + kSlots - 1) / kSlots;
  // The MFMA builtins carry no ordering of their own, so instruction
  // selection may place some of a region's MFMAs after its sched_barrier; an
  // empty asm statement that takes every accumulator (and is ordered before
  // the barrier) keeps them all inside the region.
  auto schedule_region = [&](auto id) {
    constexpr int kId = decltype(id)::value;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j) asm volatile("" ::"a"(acc[i][j]));
    sched_slots<kId, 0, kSlots, kPerSlot, kReads>();
    __builtin_amdgcn_sched_group_barrier(0x008, kMfma - kSlots, kId);
    __builtin_amdgcn_sched_barrier(0);
  };
  constexpr int kRegionLen = (WM > WN ? WM : WN) > C::kDmaA ? (WM > WN ? WM : WN) : C::kDmaA;

  // ---- epilogue ---------------------------------------------------------------
  // acc[i][j] register 4g+e holds u = 2^31 + C[row][col] (mod 2^32; the
  // accumulators start at 2^31) with
  //   row = m0 + wave_m*32*WM + 32i + (lane & 31)
  //   col = n0 + wave_n*32*WN + 32j + 8g + 4*(lane >> 5) + e.
  // Stores go through a buffer resource over the unit's tile rows, so rows
  // >= M are dropped by the range check; columns past the padded pitch (only
  // in the last tile column) get an offset beyond num_records.
  auto epilogue = [&](const Unit& U) {
    // The accumulator reads below are asm, so the compiler inserts no wait
    // states after the last MFMA for them: 24 here cover the longest
    // MFMA-write to v_accvgpr_read dependency.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    const ModulusConsts mc = pc.mod[U.plane];
    const int64_t tile_rows = min(static_cast<int64_t>(BM), args.m - U.m0);
    const uint32_t lane_off =
        static_cast<uint32_t>((wave_m * (32 * WM) + frag_row) * args.ldc + wave_n * (32 * WN) + 4 * frag_half);
    const uint32_t row_step = static_cast<uint32_t>(32 * args.ldc);
    const bool full_cols = U.n0 + BN <= args.ldc;
    // a listed unit's wave stores its quadrant only if the mask selects it
    if (kListed && ((U.quad >> (wave_m * 2 + wave_n)) & 1u) == 0u) return;
    // the unit's tile of C, or of its K slice's workspace slot
    // [slice][plane][M][ldc] (split launches never accumulate)
    int8_t* const Cp =
        args.slices <= 1
            ? base_c(U) + static_cast<int64_t>(U.plane) * args.pitch_c + U.m0 * args.ldc + U.n0
            : base_ws(U) + ((static_cast<int64_t>(U.slice) * args.nplanes + U.plane) * args.m + U.m0) * args.ldc +
                  U.n0;
    const __amdgpu_buffer_rsrc_t c_rsrc = make_rsrc(Cp, tile_rows * args.ldc - U.n0);
    const CenteredI32 kc = centered_i32_consts(mc);
    // The packed residues go through this wave's slice of the epilogue LDS
    // region (outside the stage ring, so the next unit's DMAs keep landing)
    // so the global stores are row-contiguous 16-byte chunks; kEpiParts
    // passes of WM / kEpiParts block rows each. Layout: row-major
    // kEpiRow-byte rows, 16-byte chunk c of row r at c ^ ((r >> 1) &
    // (kEpiChunks - 1)).
    int8_t* const ep = lds + C::kLds + wave * (C::kEpiBytes / C::kEpiParts);
    auto epi_swz = [](int r) { return (r >> 1) & (C::kEpiChunks - 1); };
    const int rrow = lane / C::kEpiChunks;
    const int rchunk = lane % C::kEpiChunks;
    const bool chunk_ok = full_cols || wave_n * (32 * WN) + 16 * rchunk < static_cast<int>(args.ldc - U.n0);
    constexpr int kPartRows = WM / C::kEpiParts;  // 32-row blocks per pass
#pragma unroll
    for (int part = 0; part < C::kEpiParts; ++part) {
      auto reduce = [&](auto carry, auto low_byte) {
        constexpr bool kCarry = decltype(carry)::value;
        constexpr bool kLowByte = decltype(low_byte)::value;  // m = 256: the residue is the low byte
#pragma unroll
        for (int ii = 0; ii < kPartRows; ++ii) {
          const int i = part * kPartRows + ii;
          const uint32_t off = lane_off + static_cast<uint32_t>(i) * row_step;
          uint32_t prev[WN][4];
          if constexpr (kCarry) {
            // later K block: add the centered residue carried in C (|.| <= 128)
#pragma unroll
            for (int j = 0; j < WN; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g)
                prev[j][g] = static_cast<uint32_t>(
                    __builtin_amdgcn_raw_buffer_load_b32(c_rsrc, static_cast<int>(off + 32 * j + 8 * g), 0, 0));
          }
          const int r = 32 * ii + frag_row;
#pragma unroll
          for (int j = 0; j < WN; ++j) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              uint32_t res[4];
              const Acc4 a4 = acc_read4(acc[i][j], g);
              uint32_t packed;
              if constexpr (kLowByte) {
                // 2^31 is 0 mod 256, so u's low byte is C's, read as int8 its centered residue
                packed = pack_low_bytes(a4.v[0], a4.v[1], a4.v[2], a4.v[3]);
              } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  uint32_t u = a4.v[e];
                  if constexpr (kCarry)
                    u += static_cast<uint32_t>(static_cast<int32_t>(static_cast<int8_t>(prev[j][g] >> (8 * e))));
                  res[e] = centered_residue_i32(u, mc, kc);
                }
                packed = pack_low_bytes(res[0], res[1], res[2], res[3]);
              }
              const int c = 2 * j + (g >> 1);
              *reinterpret_cast<uint32_t*>(ep + r * C::kEpiRow + ((c ^ epi_swz(r)) << 4) + 8 * (g & 1) +
                                           4 * frag_half) = packed;
            }
          }
        }
      };
      if (accumulate)
        reduce(std::true_type{}, std::false_type{});
      else if (mc.m == 256u)
        reduce(std::false_type{}, std::true_type{});
      else
        reduce(std::false_type{}, std::false_type{});
      // Read back row-contiguous: lane l takes chunk l % kEpiChunks of rows
      // q * kEpiRowsPerStore + l / kEpiChunks of this pass.
      const uint32_t goff = static_cast<uint32_t>((wave_m * (32 * WM) + 32 * kPartRows * part + rrow) * args.ldc +
                                                  wave_n * (32 * WN) + 16 * rchunk);
#pragma unroll
      for (int q = 0; q < 32 * kPartRows / C::kEpiRowsPerStore; ++q) {
        const int row = C::kEpiRowsPerStore * q + rrow;
        const v4i v = *reinterpret_cast<const v4i*>(ep + row * C::kEpiRow + ((rchunk ^ epi_swz(row)) << 4));
        const uint32_t o = goff + static_cast<uint32_t>(C::kEpiRowsPerStore * q) * static_cast<uint32_t>(args.ldc);
        __builtin_amdgcn_raw_buffer_store_b128(v, c_rsrc, static_cast<int>(chunk_ok ? o : 0x80000000u), 0, 0);
      }
    }
  };

  // ---- pipeline ----------------------------------------------------------------
  // Four LDS stages. Stream position s (the s-th K tile of this workgroup's
  // work list, across unit boundaries) is computed from stage s%4 while the
  // DMA of position s+3 into stage (s+3)%4 (last read at position s-1) is in
  // flight and the first fragments of position s+1 are prefetched. Before the
  // barrier that ends position s each wave waits until only its position s+3
  // DMAs are outstanding (older VMEM operations, the previous epilogue's
  // stores included, complete in order before them), so the barrier publishes
  // position s+2 and retires every read of stage s%4. The DMAs are issued
  // from inline asm, so the compiler tracks no LDS write for them and adds no
  // waits before the fragment reads: the explicit vmcnt waits below are what
  // orders them. They are spread over the whole step (A DMAs in the first
  // half, B DMAs in the second): each one holds the texture path for a while,
  // and bunching a step's DMAs stalls MFMA issue.
  if (u_first >= u_end) return;
  constexpr int kDmaPerTile = C::kDmaA + C::kDmaB;
  Frags f0, f1, f0n;
  issue_next(0);
  issue_next(1);
  issue_next(2);
  __builtin_amdgcn_s_waitcnt(kWaitVm[kDmaPerTile]);  // positions 0 and 1 landed
  __syncthreads();
  read_frags(0, 0, f0);
  int stage = 0;
  for (uint32_t u = u_first; u < u_end; u += u_step) {
    const Unit U = decode(u);
    if constexpr (kUniform) next_du();
    reset_acc();
    // every unit has at least one K tile (the host sizes slices so)
    uint32_t kt = 0;
    do {
      const int stage1 = (stage + 1) & 3;
      const int stage3 = (stage + 3) & 3;
      const TileSrc src = nsrc;
      // Region 1: sub-step 0 MFMAs; sub-step 1 fragment reads and the A DMAs.
#pragma unroll
      for (int t = 0; t < kRegionLen; ++t) {
        if (t < WM) f1.a[t] = read_a(stage, 1, t);
        if (t < WN) f1.b[t] = read_b(stage, 1, t);
        if (t < C::kDmaA) dma_a(src, stage3, t);
      }
      mfma_all(f0);
      schedule_region(std::integral_constant<int, 1>{});
      // Region 2: sub-step 1 MFMAs; first fragments of position s+1 and the B
      // DMAs.
#pragma unroll
      for (int t = 0; t < kRegionLen; ++t) {
        if (t < WM) f0n.a[t] = read_a(stage1, 0, t);
        if (t < WN) f0n.b[t] = read_b(stage1, 0, t);
        if (t < C::kDmaB) dma_b(src, stage3, t);
      }
      mfma_all(f1);
      // The cursor's scalar work sits in this region, where it issues in the
      // shadow of the MFMAs; after the region it would run with the MFMA
      // pipe idle.
      if constexpr (kUniform) cursor_advance(std::true_type{});
      schedule_region(std::integral_constant<int, 2>{});
      // the next position's fragments stay in this step (not sunk past the
      // cursor's branch)
#pragma unroll
      for (int i = 0; i < WM; ++i) asm volatile("" ::"v"(f0n.a[i]));
#pragma unroll
      for (int j = 0; j < WN; ++j) asm volatile("" ::"v"(f0n.b[j]));
      if constexpr (!kUniform) cursor_advance(std::false_type{});
      __builtin_amdgcn_s_waitcnt(kWaitVm[kDmaPerTile]);  // only position s+3 outstanding
      __syncthreads();
      f0 = f0n;
      stage = stage1;
    } while (++kt < U.ktiles);
    epilogue(U);
    // The first fragments of the next unit are read again here rather than
    // kept from the last step: holding them through the epilogue costs
    // registers the epilogue needs. The stage stays valid: its next DMA is
    // issued only in the next step.
    read_frags(stage, 0, f0);
  }
  __builtin_amdgcn_s_waitcnt(kWaitVm[0]);  // no DMA outlives the workgroup's LDS
}

// Zero-output tiles of a per-tile schedule: planes [0, planes) of each tile's
// rows and columns are set to 0 (reference cpu_reference.cpp:243-246). Whole
// 16-byte chunks are written: a tile's column offset is a multiple of 64, and
// the last tile column's chunks end inside the padded pitch.
__global__ __launch_bounds__(256) void zero_tiles_kernel(int8_t* c, int64_t ldc, int64_t pitch_c,
                                                         const TileFill* tiles) {
  const TileFill t = tiles[blockIdx.x];
  const uint32_t chunks = (t.cols + 15u) / 16u;
  const uint64_t per_plane = static_cast<uint64_t>(t.rows) * chunks;
  const uint64_t total = per_plane * t.planes;
  for (uint64_t i = threadIdx.x; i < total; i += blockDim.x) {
    const uint32_t p = static_cast<uint32_t>(i / per_plane);
    const uint64_t rem = i - static_cast<uint64_t>(p) * per_plane;
    const uint32_t r = static_cast<uint32_t>(rem / chunks);
    const uint32_t ch = static_cast<uint32_t>(rem - static_cast<uint64_t>(r) * chunks);
    int8_t* const dst = c + static_cast<int64_t>(p) * pitch_c + static_cast<int64_t>(t.row_off + r) * ldc + t.col_off +
                        16 * ch;
    *reinterpret_cast<v4i*>(dst) = v4i{0, 0, 0, 0};
  }
}

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* dst, uint64_t words) {
  for (uint64_t w = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; w < words;
       w += static_cast<uint64_t>(gridDim.x) * blockDim.x)
    dst[w] = 0u;
}

using CfgLarge = Cfg<4, 4>;  // 256 x 256 tiles, one workgroup per CU (all 512 registers per lane)
using CfgSmall = Cfg<2, 2>;  // 128 x 128 tiles, two workgroups per CU


template <typename Cf>
int64_t tile_count(int64_t m, int64_t n, uint32_t nplanes) {
  return ((m + Cf::BM - 1) / Cf::BM) * ((n + Cf::BN - 1) / Cf::BN) * static_cast<int64_t>(nplanes);
}

}  // namespace

GemmShape choose_gemm_shape(int64_t m, int64_t n, int64_t k, uint32_t nplanes) {
  // Results at most 16 columns wide: the skinny kernel (skinny.hip).
  GemmShape shape{};
  if (skinny_shape(m, n, k, nplanes, shape)) return shape;
  // 256 x 256 tiles when they already give every CU at least one and neither
  // side of the result is narrower than 256; otherwise 128 x 128 tiles (two
  // per CU), and split K when even those leave the chip under-filled: toward
  // ~512 units, with slices of at least 4096 K and at most 65536. Each slice
  // adds a residue tile per plane to write and sum, and short slices spend a
  // larger share in the DMA prologue and the epilogue.
  shape.tile = 128;
  shape.slices = 1;
  shape.k_slice = k;
  if (m > 128 && n > 128 && tile_count<CfgLarge>(m, n, nplanes) >= 256) {
    shape.tile = 256;
    return shape;
  }
  const int64_t tiles = tile_count<CfgSmall>(m, n, nplanes);
  if (tiles >= 256 || k < 8192) return shape;
  int64_t slices = std::min<int64_t>((512 + tiles - 1) / tiles, k / 4096);
  slices = std::max<int64_t>(slices, (k + kSafeKBlock - 1) / kSafeKBlock);
  if (slices <= 1) return shape;
  int64_t k_slice = (k + slices - 1) / slices;
  k_slice = (k_slice + CfgSmall::BK - 1) / CfgSmall::BK * CfgSmall::BK;
  slices = (k + k_slice - 1) / k_slice;
  if (slices <= 1 || slices * tiles > 0x7FFFFFFF) return shape;
  shape.slices = static_cast<uint32_t>(slices);
  shape.k_slice = k_slice;
  shape.ws_bytes = static_cast<uint64_t>(slices) * nplanes * static_cast<uint64_t>(m) * static_cast<uint64_t>(padded_ld(n));
  return shape;
}

hipError_t launch_zero_words(uint32_t* dst, uint64_t words, hipStream_t stream) {
  if (words == 0) return hipSuccess;
  if (!dst) return hipErrorInvalidValue;
  const uint64_t blocks = (words + 255) / 256;
  const unsigned grid = static_cast<unsigned>(blocks < 4096 ? blocks : 4096);
  hipLaunchKernelGGL(zero_words_kernel, dim3(grid), dim3(256), 0, stream, dst, words);
  return hipGetLastError();
}

namespace {

// Compute units of the current device (cached per device id; contexts on
// several threads may launch at once, so the cache is atomic).
int device_cu_count() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int cus = cached[dev].load(std::memory_order_relaxed);
  if (cus == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

// Ungrouped launches pass a NoTaskTable and ntasks = 1; grouped ones the
// task table and its task count (at most kMaxGroupTasks). `k_slice` is the
// K of one slice when args.slices > 1.
template <typename Cf, int kMinBlocks, bool kGrouped>
hipError_t launch_gemm_cfg(const GemmArgs& args, int64_t k_slice, const PlaneConsts& consts, hipStream_t stream,
                           const GroupArg<kGrouped>& tab, uint32_t ntasks) {
  const uint32_t tiles_m = static_cast<uint32_t>((args.m + Cf::BM - 1) / Cf::BM);
  const uint32_t tiles_n = static_cast<uint32_t>((args.ldc + Cf::BN - 1) / Cf::BN);
  const uint64_t slots = static_cast<uint64_t>(device_cu_count()) * kMinBlocks;
  // One launch per K range: the whole K split into args.slices slices, or,
  // unsplit, int32-safe blocks of 65536 whose later launches add their sum to
  // the centered residue already in C (reference cpu_reference.cpp:160-175).
  const int64_t block = args.slices > 1 ? args.k : kSafeKBlock;
  for (int64_t kb = 0; kb < args.k; kb += block) {
    const int64_t kstop = min(args.k, kb + block);
    const uint32_t accumulate = kb > 0 ? 1u : 0u;
    const int64_t ks = args.slices > 1 ? k_slice : kstop - kb;
    const uint32_t used_slices = static_cast<uint32_t>((kstop - kb + ks - 1) / ks);
    if (ks <= 0 || ks > kSafeKBlock || used_slices != args.slices) return hipErrorInvalidValue;
    const uint64_t task_units = static_cast<uint64_t>(tiles_m) * tiles_n * args.nplanes * used_slices;
    const uint64_t units = task_units * ntasks;
    if (units == 0 || units > 0x7FFFFFFFull) return hipErrorInvalidValue;
    UnitMap map{};
    map.units = static_cast<uint32_t>(units);
    map.task_units = make_div_u31(static_cast<uint32_t>(task_units));
    map.tiles_m = tiles_m;
    map.tiles = make_div_u31(tiles_m * tiles_n);
    map.planes = make_div_u31(args.nplanes);
    map.group = make_div_u31(static_cast<uint32_t>(kGroupM) * tiles_n);
    map.rows = make_div_u31(kGroupM);
    map.tail = make_div_u31(tiles_m - (tiles_m - 1) / kGroupM * kGroupM);
    map.k_begin = static_cast<uint32_t>(kb);
    map.k_stop = static_cast<uint32_t>(kstop);
    map.k_slice = static_cast<uint32_t>(ks);
    // persistent grid: one workgroup per resident slot, a multiple of 8 (one
    // share per XCD) when there are at least 8 units
    uint64_t grid = units < slots ? units : slots;
    if (grid >= 8) grid -= grid % 8;
    // every unit has the same K tiles when the slices divide the range evenly
    const bool uniform = (kstop - kb) % ks == 0;
    if (uniform)
      hipLaunchKernelGGL((plane_gemm_kernel<Cf, kMinBlocks, true, false, kGrouped>), dim3(static_cast<unsigned>(grid)),
                         dim3(kThreads), 0, stream, args, consts, map, accumulate, tab);
    else
      hipLaunchKernelGGL((plane_gemm_kernel<Cf, kMinBlocks, false, false, kGrouped>),
                         dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, stream, args, consts, map, accumulate,
                         tab);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (args.slices > 1) {
      for (uint32_t t = 0; t < ntasks; ++t) {
        int8_t* ws = args.splitk_ws;
        int8_t* c = args.c;
        if constexpr (kGrouped) {
          ws = tab.t[t].ws;
          c = tab.t[t].c;
        }
        err = launch_residue_finalize(ws, c, args.m, args.ldc, args.pitch_c, args.nplanes, args.slices, consts,
                                      stream);
        if (err != hipSuccess) return err;
      }
    }
  }
  return hipSuccess;
}

}  // namespace

namespace {

template <typename Cf, int kMinBlocks>
hipError_t launch_listed(const GemmArgs& args, const PlaneConsts& consts, const uint32_t* d_units, uint32_t units,
                         hipStream_t stream) {
  const uint64_t slots = static_cast<uint64_t>(device_cu_count()) * kMinBlocks;
  uint64_t grid = units < slots ? units : slots;
  if (grid >= 8) grid -= grid % 8;
  for (int64_t kb = 0; kb < args.k; kb += kSafeKBlock) {
    const int64_t kstop = min(args.k, kb + kSafeKBlock);
    UnitMap map{};
    map.units = units;
    map.k_begin = static_cast<uint32_t>(kb);
    map.k_stop = static_cast<uint32_t>(kstop);
    map.k_slice = static_cast<uint32_t>(kstop - kb);
    map.list = d_units;
    hipLaunchKernelGGL((plane_gemm_kernel<Cf, kMinBlocks, true, true>), dim3(static_cast<unsigned>(grid)),
                       dim3(kThreads), 0, stream, args, consts, map, kb > 0 ? 1u : 0u, NoTaskTable{});
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_gemm_listed(const GemmArgs& args, const PlaneConsts& consts, const uint32_t* d_units,
                              uint32_t units, uint32_t edge, hipStream_t stream) {
  // the list's entries are checked against the shape and edge where it is built
  if (!gemm_args_ok(args) || args.slices != 1 || !d_units || units > 0x7FFFFFFFu) return hipErrorInvalidValue;
  if (units == 0) return hipSuccess;
  if (edge == 256) return launch_listed<CfgLarge, 1>(args, consts, d_units, units, stream);
  if (edge == 128) return launch_listed<CfgSmall, 2>(args, consts, d_units, units, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_zero_tiles(int8_t* c, int64_t ldc, int64_t pitch_c, const TileFill* d_tiles, uint32_t count,
                             hipStream_t stream) {
  if (count == 0) return hipSuccess;
  if (!c || !d_tiles || ldc <= 0 || ldc % 16 || pitch_c < ldc || count > 0x7FFFFFFFu) return hipErrorInvalidValue;
  hipLaunchKernelGGL(zero_tiles_kernel, dim3(count), dim3(256), 0, stream, c, ldc, pitch_c, d_tiles);
  return hipGetLastError();
}

// ---- static scratch for calls that allocate nothing ---------------------------
// The split-K residues of rns8_mi355x_gemm_rns_noalloc live here instead of
// in a caller's workspace. Each device holds its own copy of the array for
// the life of the process. On the host the array's name is not a device
// address: host code uses the per-device address resolve_noalloc_scratch
// records (hipGetSymbolAddress with that device current).
static __device__ __align__(256) int8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<int8_t*> g_scratch[kMaxDevices] = {};
std::mutex g_scratch_mutex;
}  // namespace

hipError_t resolve_noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  if (g_scratch[device].load(std::memory_order_acquire)) return hipSuccess;
  int current = -1;
  if (hipGetDevice(&current) != hipSuccess || current != device) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[device].load(std::memory_order_acquire)) return hipSuccess;
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (!ptr || (reinterpret_cast<uintptr_t>(ptr) & 255u) != 0) return hipErrorInvalidSymbol;
  g_scratch[device].store(static_cast<int8_t*>(ptr), std::memory_order_release);
  return hipSuccess;
}

int8_t* noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  return g_scratch[device].load(std::memory_order_acquire);
}

hipError_t launch_gemm(const GemmArgs& args, const PlaneConsts& consts, hipStream_t stream) {
  if (!gemm_args_ok(args)) return hipErrorInvalidValue;
  const GemmShape shape = choose_gemm_shape(args.m, args.n, args.k, args.nplanes);
  // the workspace was sized for the plan's slices: never use a different
  // split (an unsplit call of a split shape runs unsplit where the kernel
  // allows it)
  if (args.slices > 1 && args.slices != shape.slices) return hipErrorInvalidValue;
  if (shape.tile == 16) {
    if (args.slices == shape.slices) return launch_skinny(args, shape, consts, stream);
    // an unsplit call (no workspace) of a shape the skinny kernel would
    // split: the 128 x 128 kernel, which takes any K in 65536 blocks
    if (args.slices != 1) return hipErrorInvalidValue;
    return launch_gemm_cfg<CfgSmall, 2, false>(args, args.k, consts, stream, NoTaskTable{}, 1);
  }
  if (shape.tile == 256) return launch_gemm_cfg<CfgLarge, 1, false>(args, shape.k_slice, consts, stream, NoTaskTable{}, 1);
  return launch_gemm_cfg<CfgSmall, 2, false>(args, shape.k_slice, consts, stream, NoTaskTable{}, 1);
}

hipError_t launch_gemm_grouped(const GemmArgs& shape, const PlaneConsts& consts, const TaskPtrs* tasks,
                               uint32_t count, hipStream_t stream) {
  if (!tasks || count == 0) return hipErrorInvalidValue;
  // tile and K split for the whole group (the tasks count as extra planes);
  // never more slices than the shape's own workspaces hold
  const GemmShape g = choose_gemm_shape(shape.m, shape.n, shape.k, shape.nplanes * count);
  if (g.slices > 1 && g.slices > shape.slices) return hipErrorInvalidValue;
  for (uint32_t t = 0; t < count; ++t) {
    // every task's operands pass the same checks as an ungrouped launch
    GemmArgs a = shape;
    a.a = tasks[t].a;
    a.b = tasks[t].b;
    a.c = tasks[t].c;
    a.splitk_ws = tasks[t].ws;
    a.slices = g.tile == 16 ? shape.slices : g.slices;
    if (!gemm_args_ok(a)) return hipErrorInvalidValue;
  }
  if (g.tile == 16) {
    // the skinny kernel fills the chip from one task's rows and K slices:
    // one launch per task, each with its own workspace
    for (uint32_t t = 0; t < count; ++t) {
      GemmArgs a = shape;
      a.a = tasks[t].a;
      a.b = tasks[t].b;
      a.c = tasks[t].c;
      a.splitk_ws = tasks[t].ws;
      const hipError_t err = launch_gemm(a, consts, stream);
      if (err != hipSuccess) return err;
    }
    return hipSuccess;
  }
  for (uint32_t first = 0; first < count; first += kMaxGroupTasks) {
    const uint32_t n = count - first < kMaxGroupTasks ? count - first : kMaxGroupTasks;
    TaskTable tab{};
    for (uint32_t t = 0; t < n; ++t) tab.t[t] = tasks[first + t];
    GemmArgs a = shape;
    a.a = a.b = nullptr;
    a.c = nullptr;
    a.splitk_ws = nullptr;
    a.slices = g.slices;
    const hipError_t err = g.tile == 256 ? launch_gemm_cfg<CfgLarge, 1, true>(a, g.k_slice, consts, stream, tab, n)
                                         : launch_gemm_cfg<CfgSmall, 2, true>(a, g.k_slice, consts, stream, tab, n);
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

}  // namespace rns8x
