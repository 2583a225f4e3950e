// Matrix-core rate probe for gfx950: the dense int8 MFMA rate one MI355X
// sustains on this workload's operand statistics, for the roofline context
// bench.py reports next to its measured GEMM.
//
// One 256-thread workgroup per CU; each wave keeps 16 independent 32x32
// accumulators and issues v_mfma_i32_32x32x32_i8 back to back from register
// operands, alternating between two operand sets. With `random` the operand
// bytes are a hash of the lane and register index (uniform bytes, like the
// centered residue planes); otherwise they are zero. Each workgroup records
// its elapsed shader cycles (s_memtime) and 100 MHz reference ticks
// (s_memrealtime), from which the host derives the clock the chip ran at.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t mix(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  return x ^ (x >> 16);
}

__global__ __launch_bounds__(256, 1) void mfma_rate_kernel(int iters, uint32_t random, int* sink,
                                                           unsigned long long* ticks) {
  const uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  v4i a0[4], b0[4], a1[4], b1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t s = g * 64u + 16u * i + e;
      a0[i][e] = random ? static_cast<int>(mix(s)) : 0;
      b0[i][e] = random ? static_cast<int>(mix(s + 4u)) : 0;
      a1[i][e] = random ? static_cast<int>(mix(s + 8u)) : 0;
      b1[i][e] = random ? static_cast<int>(mix(s + 12u)) : 0;
    }
  v16i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v16i{};
  __syncthreads();
  const unsigned long long c0 = __builtin_readcyclecounter();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b0[j], a0[i], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b1[j], a1[i], acc[i][j], 0, 0, 0);
  }
  const unsigned long long c1 = __builtin_readcyclecounter();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  int s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) s ^= acc[i][j][0] ^ acc[i][j][15];
  sink[g] = s;
  if (threadIdx.x == 0) {
    ticks[2 * blockIdx.x] = c1 - c0;
    ticks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

}  // namespace

// Runs `launches` probe launches of `iters` iterations after `warmup`
// untimed ones on the current device and reports the int8 rate (TOP/s, dense
// MFMA operations counted as 2 per multiply-add) and the mean shader clock
// (GHz). Returns 0, or the HIP error code.
extern "C" __attribute__((visibility("default"))) int rns8_probe_mfma_rate(int random, int iters, int warmup,
                                                                           int launches, double* tops,
                                                                           double* clock_ghz) {
  if (!tops || !clock_ghz || iters <= 0 || launches <= 0 || warmup < 0) return static_cast<int>(hipErrorInvalidValue);
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return static_cast<int>(e);
  int* sink = nullptr;
  unsigned long long* ticks = nullptr;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  auto done = [&](hipError_t err) {
    hipFree(sink);
    hipFree(ticks);
    if (t0) hipEventDestroy(t0);
    if (t1) hipEventDestroy(t1);
    return static_cast<int>(err);
  };
  if ((e = hipMalloc(&sink, static_cast<size_t>(cus) * 256 * sizeof(int))) != hipSuccess) return done(e);
  if ((e = hipMalloc(&ticks, static_cast<size_t>(cus) * 2 * sizeof(unsigned long long))) != hipSuccess) return done(e);
  if ((e = hipEventCreate(&t0)) != hipSuccess || (e = hipEventCreate(&t1)) != hipSuccess) return done(e);
  const uint32_t rnd = random ? 1u : 0u;
  for (int i = 0; i < warmup; ++i)
    hipLaunchKernelGGL(mfma_rate_kernel, dim3(cus), dim3(256), 0, nullptr, iters, rnd, sink, ticks);
  if ((e = hipGetLastError()) != hipSuccess) return done(e);
  if ((e = hipEventRecord(t0, nullptr)) != hipSuccess) return done(e);
  for (int i = 0; i < launches; ++i)
    hipLaunchKernelGGL(mfma_rate_kernel, dim3(cus), dim3(256), 0, nullptr, iters, rnd, sink, ticks);
  if ((e = hipGetLastError()) != hipSuccess) return done(e);
  if ((e = hipEventRecord(t1, nullptr)) != hipSuccess || (e = hipEventSynchronize(t1)) != hipSuccess) return done(e);
  float ms = 0.f;
  if ((e = hipEventElapsedTime(&ms, t0, t1)) != hipSuccess) return done(e);
  std::vector<unsigned long long> h(static_cast<size_t>(cus) * 2);
  if ((e = hipMemcpy(h.data(), ticks, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost)) != hipSuccess)
    return done(e);
  double ghz = 0.0;
  int n = 0;
  for (int b = 0; b < cus; ++b)
    if (h[2 * b + 1] > 0) {
      ghz += static_cast<double>(h[2 * b]) / (static_cast<double>(h[2 * b + 1]) * 10.0);  // 100 MHz ticks
      ++n;
    }
  const double ops = static_cast<double>(cus) * 4.0 * iters * 32.0 * 65536.0 * launches;
  *tops = ms > 0.f ? ops / (ms * 1e-3) / 1e12 : 0.0;
  *clock_ghz = n ? ghz / n : 0.0;
  return done(hipSuccess);
}
