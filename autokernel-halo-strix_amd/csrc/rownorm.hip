// RMSNorm and fused residual-add + RMSNorm for gfx950.
//
// Row-parallel, HBM-bound. A row is owned by TPR threads (one wave for rows
// up to 64*8 16-byte vectors, otherwise a 256- or 1024-thread workgroup).
// Each thread keeps its slice of the row in registers as fp32 between the
// sum-of-squares reduction and the normalise pass, so x and residual are read
// from HBM exactly once and new_residual / y written exactly once.
//
// Arithmetic follows reference.py:25-29 and :71-78 of the reference:
//   h     = round_T(x + residual)              (fp32 add, one rounding)
//   rms   = sqrt(sum(h^2) / cols + eps)        (fp32)
//   y     = round_T((h / rms) * weight)        (IEEE division, then multiply)
#include "ak_common.h"

namespace ak {
namespace {

template <typename T, bool RES, int VPT, int TPR>
__global__ void __launch_bounds__(TPR >= 256 ? TPR : 256)
rownorm_vec_kernel(const T* __restrict__ x, const T* __restrict__ r,
                   const T* __restrict__ w, T* __restrict__ nr, T* __restrict__ y,
                   int64_t rows, int cols, int64_t ld_x, int64_t ld_r,
                   int64_t ld_nr, int64_t ld_y, float eps) {
  constexpr int VE = Vec16<T>::VE;
  constexpr int ROWS_PER_WG = TPR >= 256 ? 1 : 256 / TPR;
  static_assert(TPR == 64 || TPR >= 256, "row owners are one wave or a whole workgroup");

  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * ROWS_PER_WG + threadIdx.x / TPR;
  if (TPR == 64 && row >= rows) return;  // whole wave leaves together
  const int nvec = cols / VE;

  const T* xr = x + row * ld_x;
  float h[VPT][VE];
  float ss = 0.0f;

#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = t + k * TPR;
    if (v < nvec) {
      Vec16<T> xv = load16(xr + (int64_t)v * VE);
      if constexpr (RES) {
        Vec16<T> rv = load16(r + row * ld_r + (int64_t)v * VE);
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          // Round the sum to T first: new_residual and the normalised value
          // both see the same rounded hidden state.
          h[k][e] = to_f32(from_f32<T>(to_f32(xv.e[e]) + to_f32(rv.e[e])));
        }
      } else {
#pragma unroll
        for (int e = 0; e < VE; ++e) h[k][e] = to_f32(xv.e[e]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < VE; ++e) h[k][e] = 0.0f;
    }
#pragma unroll
    for (int e = 0; e < VE; ++e) ss = fmaf(h[k][e], h[k][e], ss);
  }

  ss = wave_sum(ss);
  if constexpr (TPR > 64) {
    __shared__ float part[TPR / 64];
    const int wid = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 0) part[wid] = ss;
    __syncthreads();
    ss = 0.0f;
#pragma unroll
    for (int i = 0; i < TPR / 64; ++i) ss += part[i];
  }

  const float rms = sqrtf(ss / (float)cols + eps);

#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = t + k * TPR;
    if (v < nvec) {
      const int64_t off = (int64_t)v * VE;
      Vec16<T> wv = load16(w + off);
      Vec16<T> yv;
#pragma unroll
      for (int e = 0; e < VE; ++e) yv.e[e] = from_f32<T>((h[k][e] / rms) * to_f32(wv.e[e]));
      if constexpr (RES) {
        if (nr != nullptr) {
          Vec16<T> hv;
#pragma unroll
          for (int e = 0; e < VE; ++e) hv.e[e] = from_f32<T>(h[k][e]);
          store16(nr + row * ld_nr + off, hv);
        }
      }
      store16(y + row * ld_y + off, yv);
    }
  }
}

// Any width / alignment: one 256-thread workgroup per row, scalar accesses,
// the hidden state recomputed (bit-identically) in the second pass.
template <typename T, bool RES>
__global__ void __launch_bounds__(256)
rownorm_generic_kernel(const T* __restrict__ x, const T* __restrict__ r,
                       const T* __restrict__ w, T* __restrict__ nr, T* __restrict__ y,
                       int64_t rows, int cols, int64_t ld_x, int64_t ld_r,
                       int64_t ld_nr, int64_t ld_y, float eps) {
  const int64_t row = blockIdx.x;
  auto hidden = [&](int c) -> float {
    if constexpr (RES) {
      return to_f32(from_f32<T>(to_f32(x[row * ld_x + c]) + to_f32(r[row * ld_r + c])));
    } else {
      return to_f32(x[row * ld_x + c]);
    }
  };
  float ss = 0.0f;
  for (int c = threadIdx.x; c < cols; c += 256) {
    const float h = hidden(c);
    ss = fmaf(h, h, ss);
  }
  ss = wave_sum(ss);
  __shared__ float part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x / 64] = ss;
  __syncthreads();
  ss = part[0] + part[1] + part[2] + part[3];
  const float rms = sqrtf(ss / (float)cols + eps);
  for (int c = threadIdx.x; c < cols; c += 256) {
    const float h = hidden(c);
    if constexpr (RES) {
      if (nr != nullptr) nr[row * ld_nr + c] = from_f32<T>(h);
    }
    y[row * ld_y + c] = from_f32<T>((h / rms) * to_f32(w[c]));
  }
}

template <typename T, bool RES, int VPT, int TPR>
void launch_vec(const T* x, const T* r, const T* w, T* nr, T* y, int64_t rows, int cols,
                int64_t ld_x, int64_t ld_r, int64_t ld_nr, int64_t ld_y, float eps,
                hipStream_t s) {
  constexpr int ROWS_PER_WG = TPR >= 256 ? 1 : 256 / TPR;
  const int64_t grid = (rows + ROWS_PER_WG - 1) / ROWS_PER_WG;
  rownorm_vec_kernel<T, RES, VPT, TPR><<<dim3((unsigned)grid), dim3(TPR * ROWS_PER_WG), 0, s>>>(
      x, r, w, nr, y, rows, cols, ld_x, ld_r, ld_nr, ld_y, eps);
}

template <typename T, bool RES>
int dispatch(const void* xv, const void* rv, const void* wv, void* nrv, void* yv,
             int64_t rows, int64_t cols, int64_t ld_x, int64_t ld_r, int64_t ld_nr,
             int64_t ld_y, float eps, hipStream_t s, const char* name) {
  const T* x = static_cast<const T*>(xv);
  const T* r = static_cast<const T*>(rv);
  const T* w = static_cast<const T*>(wv);
  T* nr = static_cast<T*>(nrv);
  T* y = static_cast<T*>(yv);
  constexpr int VE = Vec16<T>::VE;
  bool vec_ok = cols % VE == 0 && ld_x % VE == 0 && ld_y % VE == 0 && aligned16(x) &&
                aligned16(w) && aligned16(y);
  if (RES) vec_ok = vec_ok && ld_r % VE == 0 && aligned16(r);
  if (RES && nr) vec_ok = vec_ok && ld_nr % VE == 0 && aligned16(nr);
  const int64_t nvec = cols / VE;
  const int c = (int)cols;
  if (vec_ok && nvec <= 64 * 8) {
    if (nvec <= 64) launch_vec<T, RES, 1, 64>(x, r, w, nr, y, rows, c, ld_x, ld_r, ld_nr, ld_y, eps, s);
    else if (nvec <= 128) launch_vec<T, RES, 2, 64>(x, r, w, nr, y, rows, c, ld_x, ld_r, ld_nr, ld_y, eps, s);
    else if (nvec <= 256) launch_vec<T, RES, 4, 64>(x, r, w, nr, y, rows, c, ld_x, ld_r, ld_nr, ld_y, eps, s);
    else launch_vec<T, RES, 8, 64>(x, r, w, nr, y, rows, c, ld_x, ld_r, ld_nr, ld_y, eps, s);
  } else if (vec_ok && nvec <= 256 * 8) {
    if (nvec <= 256 * 4) launch_vec<T, RES, 4, 256>(x, r, w, nr, y, rows, c, ld_x, ld_r, ld_nr, ld_y, eps, s);
    else launch_vec<T, RES, 8, 256>(x, r, w, nr, y, rows, c, ld_x, ld_r, ld_nr, ld_y, eps, s);
  } else if (vec_ok && nvec <= 1024 * 8) {
    launch_vec<T, RES, 8, 1024>(x, r, w, nr, y, rows, c, ld_x, ld_r, ld_nr, ld_y, eps, s);
  } else {
    rownorm_generic_kernel<T, RES><<<dim3((unsigned)rows), dim3(256), 0, s>>>(
        x, r, w, nr, y, rows, c, ld_x, ld_r, ld_nr, ld_y, eps);
  }
  return ak_check_launch(name);
}

int check_common(const void* x, const void* w, const void* y, int64_t rows, int64_t cols,
                 int64_t ld_x, int64_t ld_y, int dtype, const char* name) {
  if (ak_dtype_size(dtype) == 0) return ak_set_error(AK_ERR_UNSUPPORTED, "%s: unsupported dtype code %d", name, dtype);
  if (rows < 0 || cols <= 0 || cols > (int64_t)1 << 30)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: bad shape rows=%lld cols=%lld", name, (long long)rows, (long long)cols);
  if (rows > 0xFFFFFFFFll) return ak_set_error(AK_ERR_INVALID_ARG, "%s: rows=%lld exceeds 2^32-1", name, (long long)rows);
  if (ld_x < cols || ld_y < cols)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: row pitch smaller than cols", name);
  if (rows > 0 && (!x || !w || !y)) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  return AK_OK;
}

}  // namespace
}  // namespace ak

extern "C" int ak_rmsnorm_fwd(const void* x, const void* weight, void* y, int64_t rows,
                              int64_t cols, int64_t ld_x, int64_t ld_y, float eps, int dtype,
                              void* stream) {
  const char* name = "ak_rmsnorm_fwd";
  int rc = ak::check_common(x, weight, y, rows, cols, ld_x, ld_y, dtype, name);
  if (rc) return rc;
  if (rows == 0) return AK_OK;
  hipStream_t s = ak_stream(stream);
  switch (dtype) {
    case AK_DTYPE_F32: return ak::dispatch<float, false>(x, nullptr, weight, nullptr, y, rows, cols, ld_x, 0, 0, ld_y, eps, s, name);
    case AK_DTYPE_F16: return ak::dispatch<ak::f16, false>(x, nullptr, weight, nullptr, y, rows, cols, ld_x, 0, 0, ld_y, eps, s, name);
    default: return ak::dispatch<ak::bf16, false>(x, nullptr, weight, nullptr, y, rows, cols, ld_x, 0, 0, ld_y, eps, s, name);
  }
}

extern "C" int ak_fused_add_rmsnorm_fwd(const void* x, const void* residual, const void* weight,
                                        void* new_residual, void* y, int64_t rows, int64_t cols,
                                        int64_t ld_x, int64_t ld_r, int64_t ld_nr, int64_t ld_y,
                                        float eps, int dtype, void* stream) {
  const char* name = "ak_fused_add_rmsnorm_fwd";
  int rc = ak::check_common(x, weight, y, rows, cols, ld_x, ld_y, dtype, name);
  if (rc) return rc;
  if (rows > 0 && !residual) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null residual", name);
  if (ld_r < cols || (new_residual && ld_nr < cols))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: row pitch smaller than cols", name);
  if (rows == 0) return AK_OK;
  hipStream_t s = ak_stream(stream);
  switch (dtype) {
    case AK_DTYPE_F32: return ak::dispatch<float, true>(x, residual, weight, new_residual, y, rows, cols, ld_x, ld_r, ld_nr, ld_y, eps, s, name);
    case AK_DTYPE_F16: return ak::dispatch<ak::f16, true>(x, residual, weight, new_residual, y, rows, cols, ld_x, ld_r, ld_nr, ld_y, eps, s, name);
    default: return ak::dispatch<ak::bf16, true>(x, residual, weight, new_residual, y, rows, cols, ld_x, ld_r, ld_nr, ld_y, eps, s, name);
  }
}
