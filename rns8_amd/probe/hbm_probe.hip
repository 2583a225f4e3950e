// HBM stream probe for gfx950: the rate one MI355X sustains for a stream
// that reads R bytes and writes W bytes, for the roofline context bench.py
// reports next to its memory-bound stages (the pack reads 8 bytes and writes
// P per element, the export the reverse).
//
// Each thread moves four 16-byte chunks, 256 threads apart (every load and
// store instruction of a wave covers 1 KB of consecutive bytes): chunk c is
// read when c < R/16 and written when c < W/16, the written value depending
// on the read one where both exist, as in a copy. Chunks read but not
// written fold into a per-thread XOR that is stored only if it equals a
// value no fold of the source's byte pattern yields, so those loads are
// kept. A grid of independent blocks whose threads move their chunks once:
// the shape of the product's streaming kernels.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kChunksPerThread = 4;
constexpr uint32_t kThreads = 256;
constexpr uint32_t kChunksPerBlock = kChunksPerThread * kThreads;

__global__ __launch_bounds__(kThreads) void stream_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                          uint64_t read_chunks, uint64_t write_chunks,
                                                          u32x4* __restrict__ sink) {
  const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kChunksPerBlock + threadIdx.x;
  u32x4 v[kChunksPerThread];
#pragma unroll
  for (uint32_t k = 0; k < kChunksPerThread; ++k) {
    const uint64_t c = base + static_cast<uint64_t>(k) * kThreads;
    v[k] = c < read_chunks ? src[c] : u32x4{static_cast<uint32_t>(c), 0u, 0u, 0u};
  }
  u32x4 folded = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (uint32_t k = 0; k < kChunksPerThread; ++k) {
    const uint64_t c = base + static_cast<uint64_t>(k) * kThreads;
    if (c < write_chunks)
      dst[c] = v[k] ^ u32x4{1u, 2u, 3u, 4u};
    else if (c < read_chunks)
      folded ^= v[k];
  }
  // the source's bytes are all 0x5A, so a fold of any number of its chunks
  // is 0x5A5A5A5A or 0 in each word, never this value
  if (folded.x == 0x13579BDFu) sink[threadIdx.x] = folded;
}

}  // namespace

// Times `launches` stream launches (after `warmup` untimed ones) that read
// `read_bytes` and write `write_bytes` (multiples of 16, not both 0) on the
// current device, buffers allocated and filled here, and reports
// (read_bytes + write_bytes) per launch over the mean launch time, in GB/s.
// Returns 0, or the HIP error code.
extern "C" __attribute__((visibility("default"))) int rns8_probe_hbm_stream(uint64_t read_bytes, uint64_t write_bytes,
                                                                            int warmup, int launches, double* gbps) {
  if (!gbps || launches <= 0 || warmup < 0 || (read_bytes | write_bytes) % 16 != 0 ||
      (read_bytes == 0 && write_bytes == 0))
    return static_cast<int>(hipErrorInvalidValue);
  const uint64_t nr = read_bytes / 16, nw = write_bytes / 16;
  const uint64_t chunks = nr > nw ? nr : nw;
  const uint64_t blocks = (chunks + kChunksPerBlock - 1) / kChunksPerBlock;
  if (blocks > 0x7FFFFFFFull) return static_cast<int>(hipErrorInvalidValue);
  u32x4 *src = nullptr, *dst = nullptr, *sink = nullptr;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  auto done = [&](hipError_t err) {
    hipFree(src);
    hipFree(dst);
    hipFree(sink);
    if (t0) hipEventDestroy(t0);
    if (t1) hipEventDestroy(t1);
    return static_cast<int>(err);
  };
  hipError_t e = hipSuccess;
  if (nr && (e = hipMalloc(&src, read_bytes)) != hipSuccess) return done(e);
  if (nw && (e = hipMalloc(&dst, write_bytes)) != hipSuccess) return done(e);
  if ((e = hipMalloc(&sink, kThreads * sizeof(u32x4))) != hipSuccess) return done(e);
  if (nr && (e = hipMemset(src, 0x5A, read_bytes)) != hipSuccess) return done(e);
  if (nw && (e = hipMemset(dst, 0, write_bytes)) != hipSuccess) return done(e);
  if ((e = hipEventCreate(&t0)) != hipSuccess || (e = hipEventCreate(&t1)) != hipSuccess) return done(e);
  const dim3 grid(static_cast<unsigned>(blocks));
  for (int i = 0; i < warmup; ++i)
    hipLaunchKernelGGL(stream_kernel, grid, dim3(kThreads), 0, nullptr, src, dst, nr, nw, sink);
  if ((e = hipGetLastError()) != hipSuccess) return done(e);
  if ((e = hipEventRecord(t0, nullptr)) != hipSuccess) return done(e);
  for (int i = 0; i < launches; ++i)
    hipLaunchKernelGGL(stream_kernel, grid, dim3(kThreads), 0, nullptr, src, dst, nr, nw, sink);
  if ((e = hipGetLastError()) != hipSuccess) return done(e);
  if ((e = hipEventRecord(t1, nullptr)) != hipSuccess || (e = hipEventSynchronize(t1)) != hipSuccess) return done(e);
  float ms = 0.f;
  if ((e = hipEventElapsedTime(&ms, t0, t1)) != hipSuccess) return done(e);
  const double bytes = static_cast<double>(read_bytes + write_bytes) * launches;
  *gbps = ms > 0.f ? bytes / (ms * 1e-3) / 1e9 : 0.0;
  return done(hipSuccess);
}
