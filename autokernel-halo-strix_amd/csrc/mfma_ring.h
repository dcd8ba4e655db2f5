// Shared pieces of the gfx950 MFMA tile kernels (lm-head + CE forward /
// dlogits, and the lm-head gradient GEMMs): 32x32x16 MFMA wrappers, the
// global-to-LDS ring's waits and barrier, accumulator reads.
#pragma once

#include "ak_common.h"

namespace ak {

constexpr int kKB = 64;                    // K per block (one 128-byte line per bf16 row)
constexpr int kSlots = 5;                  // LDS ring slots
constexpr int kChunks = kKB / 8;           // 16-byte chunks per staged K-major row
constexpr int kSlotChunks = 256 * kChunks; // u32x4 per slot (32 KiB)
constexpr int kDma = 256 / 8 / 4;          // DMA instructions (1 KiB each) per wave per slot

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16_t mfma32(bf16, u32x4 a, u32x4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma32(f16, u32x4 a, u32x4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// s_waitcnt immediate (gfx9 encoding): vmcnt(n), expcnt and lgkmcnt(0).
constexpr int waitcnt_vm_lgkm0(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

// One accumulator element copied from its AGPR to a VGPR at this point of
// the program (an explicit read keeps the compiler from copying all 256
// accumulators into VGPRs at once ahead of the epilogue).
__device__ __forceinline__ float acc_read(float a) {
  float v;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
}

// Workgroup barrier that publishes LDS filled by this workgroup's
// global_load_lds DMA: the caller has already waited (s_waitcnt) for its own
// DMA loads. A release fence here would wait for every outstanding DMA load
// (vmcnt(0)) and so drain the ring; the empty asm statements keep the
// compiler from moving LDS accesses across the barrier instead.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// One 16-byte global-to-LDS copy per lane: lane i's 16 bytes from `src`
// land at (wave-uniform `dst` + 16 i).
__device__ __forceinline__ void dma16(const void* src, void* dst) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                   (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}

// The same copy through a buffer resource: lane i's 16 bytes at byte offset
// voff of `r` (zeros when voff is past the resource's extent).
__device__ __forceinline__ void bdma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, void* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16,
                                           voff, 0, 0, 0);
}


}  // namespace ak
