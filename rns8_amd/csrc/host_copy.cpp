// Pinned double-buffered staging for strided host matrices (host_copy.hpp).
#include "host_copy.hpp"

#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "shards.hpp"

namespace rns8x {
namespace {

// A piece of the row-major copy: rows [row0, row0 + nrows) starting at byte
// `col0` of each row, `bytes` bytes per row (a row is split only when it does
// not fit one chunk).
struct Piece {
  int64_t row0;
  int64_t nrows;
  std::size_t col0;
  std::size_t bytes;
};

std::vector<Piece> plan_pieces(std::size_t row_bytes, int64_t rows, std::size_t chunk) {
  std::vector<Piece> pieces;
  if (row_bytes <= chunk) {
    const int64_t per = static_cast<int64_t>(chunk / row_bytes);
    for (int64_t r = 0; r < rows; r += per) pieces.push_back(Piece{r, std::min(per, rows - r), 0, row_bytes});
  } else {
    for (int64_t r = 0; r < rows; ++r)
      for (std::size_t c = 0; c < row_bytes; c += chunk)
        pieces.push_back(Piece{r, 1, c, std::min(chunk, row_bytes - c)});
  }
  return pieces;
}

// Copies the rows of one piece between a strided host matrix and a packed
// buffer, on up to 8 threads for large pieces (host memory bandwidth, not one
// core's copy rate, is then the limit).
void copy_piece(const Piece& p, char* packed, char* strided, std::size_t pitch, bool to_packed) {
  const std::size_t total = static_cast<std::size_t>(p.nrows) * p.bytes;
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const int64_t threads = std::min<int64_t>({8, static_cast<int64_t>(hw), static_cast<int64_t>(total >> 21) + 1,
                                             p.nrows});
  auto run = [&](int64_t r0, int64_t r1) {
    for (int64_t r = r0; r < r1; ++r) {
      char* a = packed + static_cast<std::size_t>(r - p.row0) * p.bytes;
      char* b = strided + static_cast<std::size_t>(r) * pitch + p.col0;
      if (to_packed)
        std::memcpy(a, b, p.bytes);
      else
        std::memcpy(b, a, p.bytes);
    }
  };
  if (threads <= 1) {
    run(p.row0, p.row0 + p.nrows);
    return;
  }
  const int64_t per = (p.nrows + threads - 1) / threads;
  run_shards(static_cast<unsigned>(threads), [&](unsigned t) {
    const int64_t r0 = p.row0 + t * per, r1 = std::min(p.row0 + p.nrows, r0 + per);
    if (r0 < r1) run(r0, r1);
  });
}

}  // namespace

HostStaging::~HostStaging() {
  for (int b = 0; b < 2; ++b) {
    if (done_[b]) {
      (void)hipEventSynchronize(done_[b]);
      (void)hipEventDestroy(done_[b]);
    }
    if (buf_[b]) (void)hipHostFree(buf_[b]);
  }
}

hipError_t HostStaging::ensure() {
  for (int b = 0; b < 2; ++b) {
    if (!buf_[b]) {
      const hipError_t e = hipHostMalloc(&buf_[b], kChunkBytes, hipHostMallocDefault);
      if (e != hipSuccess) {
        buf_[b] = nullptr;
        return e;
      }
    }
    if (!done_[b]) {
      const hipError_t e = hipEventCreateWithFlags(&done_[b], hipEventDisableTiming);
      if (e != hipSuccess) {
        done_[b] = nullptr;
        return e;
      }
    }
  }
  return hipSuccess;
}

hipError_t HostStaging::to_device(void* dst, const void* src, std::size_t row_bytes, std::size_t src_pitch,
                                  int64_t rows, hipStream_t stream) {
  if (rows <= 0 || row_bytes == 0) return hipSuccess;
  std::lock_guard<std::mutex> lock(mutex_);
  hipError_t e = ensure();
  if (e != hipSuccess) return e;
  const std::vector<Piece> pieces = plan_pieces(row_bytes, rows, kChunkBytes);
  char* const d = static_cast<char*>(dst);
  for (std::size_t i = 0; i < pieces.size(); ++i) {
    const Piece& p = pieces[i];
    const int b = static_cast<int>(i & 1);
    // the DMA that last read this buffer must be finished before refilling it
    if ((e = hipEventSynchronize(done_[b])) != hipSuccess) return e;
    copy_piece(p, static_cast<char*>(buf_[b]), const_cast<char*>(static_cast<const char*>(src)), src_pitch, true);
    const std::size_t off = static_cast<std::size_t>(p.row0) * row_bytes + p.col0;
    if ((e = hipMemcpyAsync(d + off, buf_[b], static_cast<std::size_t>(p.nrows) * p.bytes, hipMemcpyHostToDevice,
                            stream)) != hipSuccess)
      return e;
    if ((e = hipEventRecord(done_[b], stream)) != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t HostStaging::to_host(void* dst, std::size_t dst_pitch, const void* src, std::size_t row_bytes,
                                int64_t rows, hipStream_t stream) {
  if (rows <= 0 || row_bytes == 0) return hipSuccess;
  std::lock_guard<std::mutex> lock(mutex_);
  hipError_t e = ensure();
  if (e != hipSuccess) return e;
  const std::vector<Piece> pieces = plan_pieces(row_bytes, rows, kChunkBytes);
  const char* const s = static_cast<const char*>(src);
  auto issue = [&](std::size_t i) -> hipError_t {
    const Piece& p = pieces[i];
    const int b = static_cast<int>(i & 1);
    const std::size_t off = static_cast<std::size_t>(p.row0) * row_bytes + p.col0;
    hipError_t err = hipMemcpyAsync(buf_[b], s + off, static_cast<std::size_t>(p.nrows) * p.bytes,
                                    hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipEventRecord(done_[b], stream);
    return err;
  };
  // the buffer for piece i+1 was last read by the host copy of piece i-1,
  // which has finished, so the next DMA is issued before copying piece i out
  if ((e = issue(0)) != hipSuccess) return e;
  for (std::size_t i = 0; i < pieces.size(); ++i) {
    if (i + 1 < pieces.size() && (e = issue(i + 1)) != hipSuccess) return e;
    const int b = static_cast<int>(i & 1);
    if ((e = hipEventSynchronize(done_[b])) != hipSuccess) return e;
    copy_piece(pieces[i], static_cast<char*>(buf_[b]), static_cast<char*>(dst), dst_pitch, false);
  }
  return hipSuccess;
}

}  // namespace rns8x
