// Direct-to-LDS operand loads shared by the gfx950 GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rns8x {

typedef int v4i __attribute__((ext_vector_type(4)));

// LDS byte address of a pointer into a __shared__ array (for M0).
__device__ __forceinline__ uint32_t lds_address(const int8_t* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) int8_t*)(const_cast<int8_t*>(p))));
}

// s_waitcnt immediates "vmcnt <= n" leaving expcnt and lgkmcnt unconstrained
// (gfx9 encoding: vmcnt[3:0] bits 3:0, expcnt bits 6:4, lgkmcnt bits 11:8,
// vmcnt[5:4] bits 15:14).
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Buffer resource word 3 for gfx9-family raw buffers (32-bit data format).
constexpr int kBufferFlags = 0x00020000;

// The same resource as four wave-uniform dwords, for the DMA asm below.
__device__ __forceinline__ v4i buffer_rsrc(const void* p, int64_t bytes) {
  const uint64_t addr = reinterpret_cast<uint64_t>(p);
  return v4i{__builtin_amdgcn_readfirstlane(static_cast<int>(addr)),
             __builtin_amdgcn_readfirstlane(static_cast<int>(addr >> 32)),
             __builtin_amdgcn_readfirstlane(static_cast<int>(bytes)), kBufferFlags};
}

// The same resource as the compiler's buffer-resource type, for the raw
// buffer load/store builtins (out-of-range dwords read as zero and are not
// written).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
  const uint64_t addr = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr >> 32));
  const int n = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
  void* const base = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(base, static_cast<short>(0), n, kBufferFlags);
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

}  // namespace rns8x
