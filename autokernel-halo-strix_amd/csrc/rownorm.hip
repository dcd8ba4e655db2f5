// RMSNorm and fused residual-add + RMSNorm for gfx950.
//
// Row-parallel, HBM-bound. A row is owned by 64..1024 threads holding one
// 16-byte vector each (up to 8 for rows over 1024 vectors). Each thread keeps
// its slice of the row in registers as fp32 between the sum-of-squares
// reduction and the normalise pass, so x and residual are read from HBM
// exactly once and new_residual / y written exactly once, with nontemporal
// (streaming) accesses.
//
// Arithmetic follows reference.py:25-29 and :71-78 of the reference:
//   h     = round_T(x + residual)              (fp32 add, one rounding)
//   rms   = sqrt(sum(h^2) / cols + eps)        (fp32)
//   y     = round_T((h / rms) * weight)        (IEEE division, then multiply)
#include "ak_common.h"

namespace ak {
namespace {

// TPR threads own a row (TPR / 64 waves; 256 / TPR rows per 256-thread
// workgroup when TPR < 256). The workgroup walks rows with a grid stride so
// the grid can be sized to the machine; the loop bound is uniform per
// workgroup, so the barrier of the multi-wave reduction is always reached by
// every wave. NT selects nontemporal (streaming) global loads and stores.
template <typename T, bool RES, int VPT, int TPR, bool NT>
__global__ void __launch_bounds__(TPR >= 256 ? TPR : 256)
rownorm_vec_kernel(const T* __restrict__ x, const T* __restrict__ r,
                   const T* __restrict__ w, T* __restrict__ nr, T* __restrict__ y,
                   int64_t rows, int cols, int64_t ld_x, int64_t ld_r,
                   int64_t ld_nr, int64_t ld_y, float eps) {
  constexpr int VE = Vec16<T>::VE;
  constexpr int RPW = TPR >= 256 ? 1 : 256 / TPR;  // rows per workgroup
  constexpr int WPR = TPR / 64;                      // waves per row
  static_assert(TPR % 64 == 0, "rows are owned by whole waves");
  __shared__ float part[RPW][WPR];

  const int t = threadIdx.x % TPR;
  const int rl = threadIdx.x / TPR;
  const int nvec = cols / VE;
  auto ld = [](const T* p) { return NT ? load16_nt(p) : load16(p); };
  auto st = [](T* p, const Vec16<T>& v) {
    if (NT) store16_nt(p, v);
    else store16(p, v);
  };

  for (int64_t base = (int64_t)blockIdx.x * RPW; base < rows; base += (int64_t)gridDim.x * RPW) {
    const int64_t row = base + rl;
    const bool live = row < rows;
    float h[VPT][VE];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = t + k * TPR;
      if (live && v < nvec) {
        Vec16<T> xv = ld(x + row * ld_x + (int64_t)v * VE);
        if constexpr (RES) {
          Vec16<T> rv = ld(r + row * ld_r + (int64_t)v * VE);
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
    if constexpr (WPR > 1) {
      if ((threadIdx.x & 63) == 0) part[rl][t / 64] = ss;
      __syncthreads();
      ss = 0.0f;
#pragma unroll
      for (int i = 0; i < WPR; ++i) ss += part[rl][i];
      __syncthreads();  // part is reused by the next row of this workgroup
    }
    const float rms = sqrtf(ss / (float)cols + eps);

#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = t + k * TPR;
      if (live && v < nvec) {
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
            st(nr + row * ld_nr + off, hv);
          }
        }
        st(y + row * ld_y + off, yv);
      }
    }
  }
}

// Any width / alignment: a 256-thread workgroup per row (rows by grid
// stride), scalar accesses, the hidden state recomputed (bit-identically) in
// the second pass.
template <typename T, bool RES>
__global__ void __launch_bounds__(256)
rownorm_generic_kernel(const T* __restrict__ x, const T* __restrict__ r,
                       const T* __restrict__ w, T* __restrict__ nr, T* __restrict__ y,
                       int64_t rows, int cols, int64_t ld_x, int64_t ld_r,
                       int64_t ld_nr, int64_t ld_y, float eps) {
  __shared__ float part[4];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
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
    if ((threadIdx.x & 63) == 0) part[threadIdx.x / 64] = ss;
    __syncthreads();
    ss = part[0] + part[1] + part[2] + part[3];
    __syncthreads();  // part is rewritten for the next row
    const float rms = sqrtf(ss / (float)cols + eps);
    for (int c = threadIdx.x; c < cols; c += 256) {
      const float h = hidden(c);
      if constexpr (RES) {
        if (nr != nullptr) nr[row * ld_nr + c] = from_f32<T>(h);
      }
      y[row * ld_y + c] = from_f32<T>((h / rms) * to_f32(w[c]));
    }
  }
}

template <typename T, bool RES, int VPT, int TPR>
void launch_vec(const T* x, const T* r, const T* w, T* nr, T* y, int64_t rows, int cols,
                int64_t ld_x, int64_t ld_r, int64_t ld_nr, int64_t ld_y, float eps,
                hipStream_t s) {
  constexpr int RPW = TPR >= 256 ? 1 : 256 / TPR;
  const unsigned grid = row_grid((rows + RPW - 1) / RPW);
  rownorm_vec_kernel<T, RES, VPT, TPR, true><<<dim3(grid), dim3(TPR * RPW), 0, s>>>(
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
#define AK_LAUNCH(VPT, TPR) launch_vec<T, RES, VPT, TPR>(x, r, w, nr, y, rows, c, ld_x, ld_r, ld_nr, ld_y, eps, s)
  // One 16-byte vector per thread while the row fits in 1024 threads: the
  // most waves in flight per byte, which is what saturates HBM here
  // (fused C3 shape: 1 vector x 512 threads beat 8 vectors x 64 threads by
  // 25% on MI355X).
  if (!vec_ok) {
    rownorm_generic_kernel<T, RES><<<dim3(row_grid(rows)), dim3(256), 0, s>>>(
        x, r, w, nr, y, rows, c, ld_x, ld_r, ld_nr, ld_y, eps);
  } else if (nvec <= 64) AK_LAUNCH(1, 64);
  else if (nvec <= 128) AK_LAUNCH(1, 128);
  else if (nvec <= 256) AK_LAUNCH(1, 256);
  else if (nvec <= 512) AK_LAUNCH(1, 512);
  else if (nvec <= 1024) AK_LAUNCH(1, 1024);
  else if (nvec <= 2048) AK_LAUNCH(2, 1024);
  else if (nvec <= 4096) AK_LAUNCH(4, 1024);
  else if (nvec <= 8192) AK_LAUNCH(8, 1024);
  else {
    rownorm_generic_kernel<T, RES><<<dim3(row_grid(rows)), dim3(256), 0, s>>>(
        x, r, w, nr, y, rows, c, ld_x, ld_r, ld_nr, ld_y, eps);
  }
#undef AK_LAUNCH
  return ak_check_launch(name);
}

int check_common(const void* x, const void* w, const void* y, int64_t rows, int64_t cols,
                 int64_t ld_x, int64_t ld_y, int dtype, const char* name) {
  if (ak_dtype_size(dtype) == 0) return ak_set_error(AK_ERR_UNSUPPORTED, "%s: unsupported dtype code %d", name, dtype);
  if (rows < 0 || cols <= 0 || cols > (int64_t)1 << 30)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: bad shape rows=%lld cols=%lld", name, (long long)rows, (long long)cols);
  if (ld_x < cols || ld_y < cols)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: row pitch smaller than cols", name);
  if (!ak_extent_ok(rows, ld_x, cols, ak_dtype_size(dtype)) || !ak_extent_ok(rows, ld_y, cols, ak_dtype_size(dtype)))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: rows=%lld x pitch exceed 64-bit addressing", name, (long long)rows);
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
  if (!ak_extent_ok(rows, ld_r, cols, ak_dtype_size(dtype)) ||
      (new_residual && !ak_extent_ok(rows, ld_nr, cols, ak_dtype_size(dtype))))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: rows=%lld x pitch exceed 64-bit addressing", name, (long long)rows);
  if (rows == 0) return AK_OK;
  hipStream_t s = ak_stream(stream);
  switch (dtype) {
    case AK_DTYPE_F32: return ak::dispatch<float, true>(x, residual, weight, new_residual, y, rows, cols, ld_x, ld_r, ld_nr, ld_y, eps, s, name);
    case AK_DTYPE_F16: return ak::dispatch<ak::f16, true>(x, residual, weight, new_residual, y, rows, cols, ld_x, ld_r, ld_nr, ld_y, eps, s, name);
    default: return ak::dispatch<ak::bf16, true>(x, residual, weight, new_residual, y, rows, cols, ld_x, ld_r, ld_nr, ld_y, eps, s, name);
  }
}
