// Buffer-resource access shared by the Mamba-1 scan kernels with whole-tile
// layouts (selective_scan.hip's forward, selective_scan_bwd_fast.hip's
// reverse pass): wave-uniform resources based at a workgroup's first row,
// fixed per-lane 32-bit offsets, and the tile offset in the scalar offset.
// Accesses outside a resource's extent read 0 and drop stores (hardware range
// checking), so a clamped tile index is always a valid load.
#pragma once

#include "scan_common.h"

namespace ak {

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t Rsrc;

// Raw bits of 4 consecutive elements of T.
template <typename T>
using Raw4 = std::conditional_t<sizeof(T) == 4, u32x4, u32x2>;
// Raw bits of one element of T.
template <typename T>
using Raw1 = std::conditional_t<sizeof(T) == 4, uint32_t, uint16_t>;

// Buffer resource over `bytes` bytes at `base` (raw, unswizzled; gfx9 data
// format field as used for untyped buffer access).
__device__ __forceinline__ Rsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

template <typename T>
__device__ __forceinline__ Raw4<T> bload4(Rsrc r, uint32_t voff, uint32_t soff) {
  if constexpr (sizeof(T) == 4)
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
  else
    return __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0);
}

template <typename T>
__device__ __forceinline__ Raw1<T> bload1(Rsrc r, uint32_t voff, uint32_t soff) {
  if constexpr (sizeof(T) == 4)
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
  else
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 0);
}

template <typename T>
__device__ __forceinline__ float raw_f32(Raw1<T> v) {
  return to_f32(__builtin_bit_cast(T, v));
}

// Element k (compile-time after unrolling) of a Raw4 as fp32.
template <typename T>
__device__ __forceinline__ float raw4_f32(const Raw4<T>& v, int k) {
  if constexpr (sizeof(T) == 4) {
    // the element goes through a scalar first: hipcc (ROCm 7.2) folds a
    // __builtin_bit_cast of an ext_vector element to element 0 for every k
    const uint32_t w = v[k];
    return __builtin_bit_cast(float, w);
  } else {
    const uint32_t w = v[k >> 1];
    return raw_f32<T>((uint16_t)((k & 1) ? (w >> 16) : (w & 0xFFFFu)));
  }
}

template <typename T>
__device__ __forceinline__ void bstore1(Rsrc r, uint32_t voff, float v) {
  if constexpr (sizeof(T) == 4)
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, (int)voff, 0, 0);
  else
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, from_f32<T>(v)), r, (int)voff, 0, 0);
}

// Four consecutive elements of T from a float4 (one 16- or 8-byte store),
// the tile offset in the scalar offset.
template <typename T>
__device__ __forceinline__ void bstore4_at(Rsrc r, uint32_t voff, uint32_t soff, float4 v) {
  if constexpr (sizeof(T) == 4) {
    const u32x4 w = {__builtin_bit_cast(uint32_t, v.x), __builtin_bit_cast(uint32_t, v.y),
                     __builtin_bit_cast(uint32_t, v.z), __builtin_bit_cast(uint32_t, v.w)};
    __builtin_amdgcn_raw_buffer_store_b128(w, r, (int)voff, (int)soff, 0);
  } else {
    auto bits = [](float f) { return (uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(f)); };
    const u32x2 w = {bits(v.x) | (bits(v.y) << 16), bits(v.z) | (bits(v.w) << 16)};
    __builtin_amdgcn_raw_buffer_store_b64(w, r, (int)voff, (int)soff, 0);
  }
}

// bstore1 with the tile offset in the scalar offset.
template <typename T>
__device__ __forceinline__ void bstore1_at(Rsrc r, uint32_t voff, uint32_t soff, float v) {
  if constexpr (sizeof(T) == 4)
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, (int)voff, (int)soff, 0);
  else
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, from_f32<T>(v)), r, (int)voff,
                                          (int)soff, 0);
}

}  // namespace ak
