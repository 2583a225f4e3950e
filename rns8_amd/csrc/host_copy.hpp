// Host <-> device transfers of row-strided matrices through pinned staging.
//
// The C ABI takes pageable host memory with an arbitrary row stride. Copying
// that with hipMemcpy2DAsync runs one DMA per row; instead, rows are gathered
// into (or scattered from) two pinned staging buffers by host threads while
// the DMA engine drains (or fills) the other buffer, so the PCIe link sees
// large contiguous transfers and host copying overlaps them.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <mutex>

namespace rns8x {

class HostStaging {
 public:
  static constexpr std::size_t kChunkBytes = std::size_t{16} << 20;

  HostStaging() = default;
  HostStaging(const HostStaging&) = delete;
  HostStaging& operator=(const HostStaging&) = delete;
  ~HostStaging();

  // dst (device) receives `rows` rows of `row_bytes` bytes, packed
  // contiguously; row r is read from src + r * src_pitch. Enqueued on
  // `stream`; returns after the last host copy, the DMA may still run.
  hipError_t to_device(void* dst, const void* src, std::size_t row_bytes, std::size_t src_pitch, int64_t rows,
                       hipStream_t stream);

  // dst (host) row r at dst + r * dst_pitch receives row r of the packed
  // device matrix src. Returns when dst holds the data.
  hipError_t to_host(void* dst, std::size_t dst_pitch, const void* src, std::size_t row_bytes, int64_t rows,
                     hipStream_t stream);

 private:
  hipError_t ensure();

  std::mutex mutex_;
  void* buf_[2] = {nullptr, nullptr};
  hipEvent_t done_[2] = {nullptr, nullptr};
};

}  // namespace rns8x
