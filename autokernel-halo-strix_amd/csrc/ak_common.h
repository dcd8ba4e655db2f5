// Shared device helpers for the gfx950 kernel library: element types,
// 16-byte vector I/O, wave64 DPP reductions and the C-ABI error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <type_traits>

#include "autokernel_mi355x.h"

namespace ak {

typedef __bf16 bf16;
typedef _Float16 f16;

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------
// Element conversion. float -> f16 / bf16 conversions round to nearest even
// (v_cvt_f16_f32 / v_cvt_pk_bf16_f32 on gfx950).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(f16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(bf16 v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) { return (f16)v; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) { return (bf16)v; }

// Two floats as a packed pair of 16-bit T (a in the low half), rounded to
// nearest even as from_f32 does, in one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32.
// (Two scalar conversions joined by a shift and an or take three instructions:
// the compiler converts each half separately.)
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef f16 f16x2_t __attribute__((ext_vector_type(2)));
template <typename T> __device__ __forceinline__ uint32_t pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2<bf16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
template <> __device__ __forceinline__ uint32_t pack2<f16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, f16x2_t));
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// One 16-byte global access viewed as VE elements of T.
template <typename T>
union Vec16 {
  static constexpr int VE = 16 / sizeof(T);
  u32x4 u;
  T e[VE];
};

template <typename T>
__device__ __forceinline__ Vec16<T> load16(const T* p) {
  Vec16<T> v;
  v.u = *reinterpret_cast<const u32x4*>(p);
  return v;
}

template <typename T>
__device__ __forceinline__ Vec16<T> load16_nt(const T* p) {
  Vec16<T> v;
  v.u = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return v;
}

template <typename T>
__device__ __forceinline__ void store16(T* p, const Vec16<T>& v) {
  *reinterpret_cast<u32x4*>(p) = v.u;
}

template <typename T>
__device__ __forceinline__ void store16_nt(T* p, const Vec16<T>& v) {
  __builtin_nontemporal_store(v.u, reinterpret_cast<u32x4*>(p));
}

// ---------------------------------------------------------------------------
// Wave64 reductions. Within a 16-lane row the partner values come from DPP
// lane permutations (quad_perm xor1 / xor2, row_half_mirror, row_mirror);
// across the four rows from xor shuffles (ds_bpermute). Every lane ends with
// the full result.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within 16

__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  return v;
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  v += __shfl_xor(v, 16, kWave);
  v += __shfl_xor(v, 32, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  v = fmaxf(v, __shfl_xor(v, 32, kWave));
  return v;
}

// exp(x) through the hardware base-2 exponential. exp(-inf) = 0 exactly.
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * kLog2e);
}

// Natural logarithm through the hardware base-2 logarithm.
__device__ __forceinline__ float fast_log(float x) {
  return __builtin_amdgcn_logf(x) * kLn2;
}

// tanh(a) = sign(a) * (1 - e) / (1 + e) with e = exp(-2|a|); saturates to
// +-1 for large |a| and is exact at 0.
__device__ __forceinline__ float tanh_f32(float a) {
  float e = fast_exp(-2.0f * fabsf(a));
  float r = (1.0f - e) / (1.0f + e);
  return copysignf(r, a);
}

// Grid cap of the row kernels. They walk their rows (or row groups) with a
// workgroup-uniform grid stride, so any row count runs on a grid of at most
// this many workgroups: 2^20 workgroups x 1024 threads stays inside HIP's
// 2^32 work-items per launch dimension and still fills all 256 CUs many
// times over.
constexpr int64_t kMaxRowGrid = (int64_t)1 << 20;

inline unsigned row_grid(int64_t units) {
  return (unsigned)(units < kMaxRowGrid ? units : kMaxRowGrid);
}

__host__ __device__ inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Compute units of the current device (queried once per device; ak_capi.hip).
int cu_count();

}  // namespace ak

// ---------------------------------------------------------------------------
// Host-side error plumbing shared by every entry point (defined in ak_capi.hip).
// ---------------------------------------------------------------------------
int ak_set_error(int code, const char* fmt, ...);
int ak_check_launch(const char* what);

inline hipStream_t ak_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Whether rows x pitch elements of esz bytes (the last row only `cols` long)
// stay addressable with signed 64-bit byte offsets.
inline bool ak_extent_ok(int64_t rows, int64_t pitch, int64_t cols, int esz) {
  const int64_t lim = INT64_MAX / (esz > 0 ? esz : 1);
  if (rows <= 1 || pitch <= 0) return cols <= lim;
  return pitch <= lim && cols <= lim && (rows - 1) <= (lim - cols) / pitch;
}

inline int ak_dtype_size(int dtype) {
  return dtype == AK_DTYPE_F32 ? 4 : (dtype == AK_DTYPE_F16 || dtype == AK_DTYPE_BF16) ? 2 : 0;
}
