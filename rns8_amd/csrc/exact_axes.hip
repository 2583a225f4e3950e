// Exact-wide magnitude proofs on the device (reference
// src/core/exact_range.hpp:34-157, api_gemm.cpp:870-874):
//
// * native_axes: the per-row and per-column summaries of a 64-bit operand at
//   pack time. Pass 1 stages 64 x 64 tiles in LDS; two waves summarize the
//   tile's rows (each over half of its columns) and two its columns, and
//   each tile stores one partial per row and per column (plain stores into
//   the matrix's partial scratch, no atomics). A finishing launch merges
//   each axis's partials into its record and takes the operand's max |x|
//   (one atomic max per block). Pass 2, once every centre is known, does the
//   same for the deviation sums around each axis's centre.
// * product_axes: the cell bounds of C = A x B from A's row records and B's
//   column records, reduced per row (one wave per row) and per column (one
//   wave per column), and C's bound min(k maxA maxB, max cell).
// * proof_snapshot: the records and maxima a GEMM result keeps until its own
//   summaries are needed.
//
// The arithmetic is exact_axes.hpp's, shared with the host tests.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "exact_axes.hpp"
#include "kernels.hpp"

namespace rns8x {
namespace {

using namespace xa;

constexpr int kTile = 64;
constexpr int64_t kMaxGridY = 65535;
// Elements of a half-tile run read per batch: the batch's LDS reads issue
// together and one wait covers them (a rolled loop waits on every read).
constexpr int kWalkBatch = 8;

// f(elem(j)) for j in [j0, j1): whole 32-element runs (every run of a full
// tile) in batches of kWalkBatch reads, ragged ones one element at a time.
template <typename E, typename F>
__device__ __forceinline__ void walk_run(int j0, int j1, E elem, F f) {
  if (j1 - j0 == kTile / 2) {
#pragma unroll 1
    for (int b = 0; b < kTile / 2; b += kWalkBatch) {
      u64 v[kWalkBatch];
#pragma unroll
      for (int e = 0; e < kWalkBatch; ++e) v[e] = elem(j0 + b + e);
#pragma unroll
      for (int e = 0; e < kWalkBatch; ++e) f(v[e]);
    }
  } else {
    for (int j = j0; j < j1; ++j) f(elem(j));
  }
}

// One pass over the 64 x 64 tiles of a rows x cols operand (row stride ld).
// Block (x, y) takes tile column x and tile rows y, y + gridDim.y, ...; each
// lane holds its 16 elements of the next tile in registers, loaded while the
// current tile is summarized. Partials: row r of tile column x at
// row_part[x * rows + r], column c of tile row y at col_part[y * cols + c].
// Pass 1 (Dev = false) also clears the result's 8 proof words (block (0,
// 0)), which the finishing launch fills; pass 2 reads the axis centres from
// the records pass 1 finished.
template <bool Signed, bool Dev>
__global__ __launch_bounds__(256) void native_axes_pass(const uint64_t* __restrict__ src, int64_t rows, int64_t cols,
                                                       int64_t ld, AxisPartial* __restrict__ row_part,
                                                       AxisPartial* __restrict__ col_part,
                                                       const AxisRecord* __restrict__ row_rec,
                                                       const AxisRecord* __restrict__ col_rec, u64* __restrict__ words) {
  // the tile as 32-bit halves at a row stride of 65 words: row and column
  // reads are both free of bank conflicts
  __shared__ uint32_t tile_lo[kTile][kTile + 1], tile_hi[kTile][kTile + 1];
  __shared__ AxisPartial second[2][kTile];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kTile;
  const int nc = static_cast<int>(cols - c0 < kTile ? cols - c0 : kTile);
  if (!Dev && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < 8) words[threadIdx.x] = 0;
  // waves 0, 1: rows (lane = row) over column halves; waves 2, 3: columns
  // (lane = column) over row halves
  const bool by_row = wave < 2;
  const int half = wave & 1;
  i128 col_centre = 0;
  if (Dev && !by_row && lane < nc) col_centre = record_centre(col_rec[c0 + lane]);
  const int64_t tiles_y = (rows + kTile - 1) / kTile;
  // rows wave, wave + 4, ..., wave + 60 of a tile, column c0 + lane
  u64 next[kTile / 4];
  auto fetch = [&](int64_t ty) {
    const int64_t r0 = ty * kTile;
    const int nr = static_cast<int>(rows - r0 < kTile ? rows - r0 : kTile);
#pragma unroll
    for (int q = 0; q < kTile / 4; ++q) {
      const int i = wave + 4 * q;
      next[q] = lane < nc && i < nr ? src[(r0 + i) * ld + c0 + lane] : 0;
    }
  };
  if (static_cast<int64_t>(blockIdx.y) < tiles_y) fetch(blockIdx.y);
  for (int64_t ty = blockIdx.y; ty < tiles_y; ty += gridDim.y) {
    const int64_t r0 = ty * kTile;
    const int nr = static_cast<int>(rows - r0 < kTile ? rows - r0 : kTile);
    __syncthreads();  // the previous tile's readers are done
#pragma unroll
    for (int q = 0; q < kTile / 4; ++q) {
      tile_lo[wave + 4 * q][lane] = static_cast<uint32_t>(next[q]);
      tile_hi[wave + 4 * q][lane] = static_cast<uint32_t>(next[q] >> 32);
    }
    __syncthreads();
    if (ty + gridDim.y < tiles_y) fetch(ty + gridDim.y);
    const int axes = by_row ? nr : nc, len = by_row ? nc : nr;
    const int j0 = half * 32, j1 = j0 + 32 < len ? j0 + 32 : len;
    AxisPartial p = empty_partial();
    auto row_elem = [&](int j) { return (static_cast<u64>(tile_hi[lane][j]) << 32) | tile_lo[lane][j]; };
    auto col_elem = [&](int j) { return (static_cast<u64>(tile_hi[j][lane]) << 32) | tile_lo[j][lane]; };
    if (lane < axes) {
      if (!Dev) {
        PartialAcc acc;
        if (by_row)
          walk_run(j0, j1, row_elem, [&](u64 x) { acc.add(x, Signed); });
        else
          walk_run(j0, j1, col_elem, [&](u64 x) { acc.add(x, Signed); });
        p = acc.partial();
      } else {
        const i128 centre = by_row ? record_centre(row_rec[r0 + lane]) : col_centre;
        DeviationAcc acc;
        if (by_row)
          walk_run(j0, j1, row_elem, [&](u64 x) { acc.add(deviation(x, centre, Signed)); });
        else
          walk_run(j0, j1, col_elem, [&](u64 x) { acc.add(deviation(x, centre, Signed)); });
        p.sum = acc.value();
      }
    }
    if (half == 1) second[by_row ? 0 : 1][lane] = p;
    __syncthreads();
    if (half == 0 && lane < axes) {
      partial_merge(p, second[by_row ? 0 : 1][lane]);
      if (by_row)
        row_part[static_cast<int64_t>(blockIdx.x) * rows + r0 + lane] = p;
      else
        col_part[ty * cols + c0 + lane] = p;
    }
  }
}

// Merges each axis's partials (rows first, then columns): pass 1 writes the
// records and the operand's max |x| (words[0], an atomic max per block);
// pass 2 adds the deviation sums. A block takes 32 axes; its 8 thread groups
// each merge every 8th partial of them, and group 0 merges the 8 results.
template <bool Signed, bool Dev>
__global__ __launch_bounds__(256) void native_axes_finish(const AxisPartial* __restrict__ row_part,
                                                          const AxisPartial* __restrict__ col_part, int64_t rows,
                                                          int64_t cols, AxisRecord* __restrict__ out_rows,
                                                          AxisRecord* __restrict__ out_cols, u64* __restrict__ words) {
  constexpr int kAxes = 32, kGroups = 8;
  __shared__ AxisPartial part_of[kGroups][kAxes];
  __shared__ u64 block_max;
  const int64_t tiles_x = (cols + kTile - 1) / kTile, tiles_y = (rows + kTile - 1) / kTile;
  const int a = threadIdx.x % kAxes, g = threadIdx.x / kAxes;
  if (threadIdx.x == 0) block_max = 0;
  u64 best = 0;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kAxes; base < rows + cols;
       base += static_cast<int64_t>(gridDim.x) * kAxes) {
    const int64_t i = base + a;
    const bool valid = i < rows + cols, is_row = i < rows;
    const int64_t axis = is_row ? i : i - rows, stride = is_row ? rows : cols, parts = is_row ? tiles_x : tiles_y;
    AxisPartial p = empty_partial();
    if (valid) {
      const AxisPartial* const part = (is_row ? row_part : col_part) + axis;
      for (int64_t t = g; t < parts; t += kGroups) {
        if (!Dev)
          partial_merge(p, part[t * stride]);
        else
          p.sum += part[t * stride].sum;
      }
    }
    __syncthreads();  // the previous round's readers are done
    part_of[g][a] = p;
    __syncthreads();
    if (g == 0 && valid) {
      for (int h = 1; h < kGroups; ++h) {
        if (!Dev)
          partial_merge(p, part_of[h][a]);
        else
          p.sum += part_of[h][a].sum;
      }
      AxisRecord* const rec = (is_row ? out_rows : out_cols) + axis;
      if (!Dev) {
        // the groups' partials start empty (hi = not_lo = 0 are neutral)
        const AxisRecord r = native_record(p, static_cast<u64>(is_row ? cols : rows), Signed);
        *rec = r;
        if (is_row) best = r.max_magnitude[0] > best ? r.max_magnitude[0] : best;
      } else {
        put_u128(rec->deviation_sum, p.sum);
      }
    }
  }
  if (!Dev) {
    if (best) atomicMax(reinterpret_cast<unsigned long long*>(&block_max), static_cast<unsigned long long>(best));
    __syncthreads();
    if (threadIdx.x == 0 && block_max)
      atomicMax(reinterpret_cast<unsigned long long*>(words), static_cast<unsigned long long>(block_max));
  }
}

struct ProductArgs {
  const AxisRecord* arows;  // m records (unused for a uniform A)
  const AxisRecord* bcols;  // n records (unused for a uniform B)
  AxisKind akind, bkind;
  const u64* amax;  // 4 words: A's bound
  const u64* bmax;  // 4 words: B's bound
  int64_t m, n;
  u64 k;
  AxisRecord* out_rows;
  AxisRecord* out_cols;
  u64* out_words;
};

__device__ __forceinline__ void wave_reduce(U256& mx, U256& sm) {
  for (int off = 32; off > 0; off >>= 1) {
    U256 om, os;
    for (int i = 0; i < 4; ++i) {
      om.w[i] = __shfl_xor(mx.w[i], off);
      os.w[i] = __shfl_xor(sm.w[i], off);
    }
    mx = max256(mx, om);
    sm = sat_add(sm, os);
  }
}

__device__ __forceinline__ void write_carried(AxisRecord* out, const U256& mx, const U256& sm) {
  AxisRecord r{};
  put_u256(r.max_magnitude, mx);
  put_u256(r.absolute_sum, sm);
  *out = r;
}

// Rows == true: one wave per row r of C, lanes over the columns; false: one
// wave per column, lanes over the rows. Each wave writes its axis's maximum
// and (saturating) sum of cell bounds.
template <bool Rows>
__global__ __launch_bounds__(256) void product_axes_kernel(ProductArgs p) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (blockDim.x >> 6);
  const int64_t outer = Rows ? p.m : p.n, inner = Rows ? p.n : p.m;
  const AxisKind fixed_kind = Rows ? p.akind : p.bkind, var_kind = Rows ? p.bkind : p.akind;
  const AxisRecord* const fixed_recs = Rows ? p.arows : p.bcols;
  const AxisRecord* const var_recs = Rows ? p.bcols : p.arows;
  const U256 fixed_max = get_u256(Rows ? p.amax : p.bmax), var_max = get_u256(Rows ? p.bmax : p.amax);
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6); o < outer;
       o += waves) {
    const AxisTerms fixed = axis_terms(fixed_kind == AxisKind::Uniform ? nullptr : fixed_recs + o, fixed_kind,
                                       fixed_max, p.k);
    U256 mx = zero256(), sm = zero256();
    for (int64_t i = lane; i < inner; i += 64) {
      const AxisTerms var = axis_terms(var_kind == AxisKind::Uniform ? nullptr : var_recs + i, var_kind, var_max,
                                       p.k);
      const U256 cell = Rows ? cell_bound(fixed, var) : cell_bound(var, fixed);
      mx = max256(mx, cell);
      sm = sat_add(sm, cell);
    }
    wave_reduce(mx, sm);
    if (lane == 0) write_carried(Rows ? p.out_rows + o : p.out_cols + o, mx, sm);
  }
}

// C's bound: min(k maxA maxB, max over the row maxima); one block.
__global__ __launch_bounds__(256) void product_bound_kernel(ProductArgs p) {
  __shared__ U256 part[4];
  U256 mx = zero256();
  for (int64_t r = threadIdx.x; r < p.m; r += blockDim.x) mx = max256(mx, get_u256(p.out_rows[r].max_magnitude));
  for (int off = 32; off > 0; off >>= 1) {
    U256 o;
    for (int i = 0; i < 4; ++i) o.w[i] = __shfl_xor(mx.w[i], off);
    mx = max256(mx, o);
  }
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) mx = max256(mx, part[w]);
    const U256 outer = sat_mul(sat_mul64(p.k, get_u256(p.amax)), get_u256(p.bmax));
    put_u256(p.out_words, min256(outer, mx));
    put_u256(p.out_words + 4, zero256());
  }
}

// A result's lazy proof: A's row records, B's column records, maxA into
// words[0..3] and maxB into words[4..7].
__global__ __launch_bounds__(256) void proof_snapshot_kernel(const uint4* __restrict__ arows,
                                                             const uint4* __restrict__ bcols,
                                                             const u64* __restrict__ a_words,
                                                             const u64* __restrict__ b_words, int64_t m_chunks,
                                                             int64_t n_chunks, uint4* __restrict__ out_rows,
                                                             uint4* __restrict__ out_cols, u64* __restrict__ words) {
  const int64_t total = m_chunks + n_chunks;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (i < m_chunks) out_rows[i] = arows[i];
    else out_cols[i - m_chunks] = bcols[i - m_chunks];
  }
  if (blockIdx.x == 0 && threadIdx.x < 8) words[threadIdx.x] = threadIdx.x < 4 ? a_words[threadIdx.x] : b_words[threadIdx.x - 4];
}

unsigned blocks_for(int64_t items, int64_t per_block, int64_t cap) {
  int64_t b = (items + per_block - 1) / per_block;
  if (b < 1) b = 1;
  if (b > cap) b = cap;
  return static_cast<unsigned>(b);
}

}  // namespace

hipError_t launch_native_axes(const void* src, int64_t rows, int64_t cols, int64_t ld, bool is_signed,
                              xa::AxisPartial* row_part, xa::AxisPartial* col_part, xa::AxisRecord* out_rows,
                              xa::AxisRecord* out_cols, uint64_t* words, hipStream_t stream) {
  if (!src || !row_part || !col_part || !out_rows || !out_cols || !words || rows <= 0 || cols <= 0 || ld < cols)
    return hipErrorInvalidValue;
  const int64_t tiles_x = (cols + kTile - 1) / kTile, tiles_y = (rows + kTile - 1) / kTile;
  if (tiles_x > 0x7FFFFFFFll) return hipErrorInvalidValue;
  // two tiles per block where there are enough: one loads while the other is summarized
  const int64_t gy = tiles_x * tiles_y >= 2048 ? (tiles_y + 1) / 2 : tiles_y;
  const dim3 grid(static_cast<unsigned>(tiles_x), static_cast<unsigned>(gy < kMaxGridY ? gy : kMaxGridY));
  const uint64_t* s = static_cast<const uint64_t*>(src);
  const unsigned fin = blocks_for(rows + cols, 32, 4096);
  auto run = [&](auto sgn) {
    constexpr bool S = decltype(sgn)::value;
    hipLaunchKernelGGL((native_axes_pass<S, false>), grid, dim3(256), 0, stream, s, rows, cols, ld, row_part,
                       col_part, out_rows, out_cols, words);
    hipLaunchKernelGGL((native_axes_finish<S, false>), dim3(fin), dim3(256), 0, stream, row_part, col_part, rows,
                       cols, out_rows, out_cols, words);
    hipLaunchKernelGGL((native_axes_pass<S, true>), grid, dim3(256), 0, stream, s, rows, cols, ld, row_part,
                       col_part, out_rows, out_cols, words);
    hipLaunchKernelGGL((native_axes_finish<S, true>), dim3(fin), dim3(256), 0, stream, row_part, col_part, rows,
                       cols, out_rows, out_cols, words);
  };
  if (is_signed)
    run(std::true_type{});
  else
    run(std::false_type{});
  return hipGetLastError();
}

hipError_t launch_product_axes(const xa::AxisRecord* arows, uint32_t akind, const xa::AxisRecord* bcols,
                               uint32_t bkind, const uint64_t* a_words, const uint64_t* b_words, int64_t m,
                               int64_t n, uint64_t k, xa::AxisRecord* out_rows, xa::AxisRecord* out_cols,
                               uint64_t* out_words, hipStream_t stream) {
  if (akind > 2 || bkind > 2 || m <= 0 || n <= 0 || k == 0 || !out_rows || !out_cols || !out_words || !a_words ||
      !b_words || (akind != 2 && !arows) || (bkind != 2 && !bcols))
    return hipErrorInvalidValue;
  const ProductArgs p{arows, bcols, static_cast<AxisKind>(akind), static_cast<AxisKind>(bkind), a_words, b_words,
                      m, n, k, out_rows, out_cols, out_words};
  // four waves per block, one axis per wave
  hipLaunchKernelGGL(product_axes_kernel<true>, dim3(blocks_for(m, 4, 8192)), dim3(256), 0, stream, p);
  hipLaunchKernelGGL(product_axes_kernel<false>, dim3(blocks_for(n, 4, 8192)), dim3(256), 0, stream, p);
  hipLaunchKernelGGL(product_bound_kernel, dim3(1), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_proof_snapshot(const xa::AxisRecord* arows, const xa::AxisRecord* bcols, const uint64_t* a_words,
                                 const uint64_t* b_words, int64_t m, int64_t n, xa::AxisRecord* out_rows,
                                 xa::AxisRecord* out_cols, uint64_t* out_words, hipStream_t stream) {
  if (!a_words || !b_words || !out_words || m < 0 || n < 0 || (m && (!arows || !out_rows)) ||
      (n && (!bcols || !out_cols)))
    return hipErrorInvalidValue;
  constexpr int64_t kChunks = sizeof(xa::AxisRecord) / sizeof(uint4);
  hipLaunchKernelGGL(proof_snapshot_kernel, dim3(blocks_for((m + n) * kChunks, 256, 2048)), dim3(256), 0, stream,
                     reinterpret_cast<const uint4*>(arows), reinterpret_cast<const uint4*>(bcols), a_words, b_words,
                     m * kChunks, n * kChunks, reinterpret_cast<uint4*>(out_rows), reinterpret_cast<uint4*>(out_cols),
                     out_words);
  return hipGetLastError();
}

}  // namespace rns8x
