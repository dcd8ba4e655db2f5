// Row softmax over the last dimension for gfx950 (reference.py:14-17).
//
// HBM-bound: each row is read once into registers (as fp32), reduced for its
// max and for sum(exp(x - max)) with wave64 DPP reductions, then normalised
// and written once, with nontemporal accesses. Rows of up to 128 16-byte
// vectors are owned by one wave (no barriers), wider rows by up to 1024
// threads holding one vector each (up to 8 past 1024 vectors). Rows are
// indexed with 64-bit arithmetic and walked by grid stride on a capped grid,
// so every row is written whatever the row count.
//
// -inf logits give exp2(-inf) = 0 exactly; a row with a single finite entry
// returns exactly 1.0 there. The file is built without fast-math so those
// IEEE special cases are honoured.
#include "ak_common.h"

namespace ak {
namespace {

// TPR threads own a row (TPR / 64 waves; 256 / TPR rows per workgroup when
// TPR < 256); rows are walked with a workgroup-uniform grid stride so the
// cross-wave reductions' barriers are reached by every wave. NT selects
// nontemporal global loads and stores.
template <typename T, int VPT, int TPR, bool NT>
__global__ void __launch_bounds__(TPR >= 256 ? TPR : 256)
softmax_vec_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t rows, int cols,
                   int64_t ld_x, int64_t ld_y) {
  constexpr int VE = Vec16<T>::VE;
  constexpr int RPW = TPR >= 256 ? 1 : 256 / TPR;
  constexpr int WPR = TPR / 64;
  static_assert(TPR % 64 == 0, "rows are owned by whole waves");
  __shared__ float part[RPW][WPR];
  const int t = threadIdx.x % TPR;
  const int rl = threadIdx.x / TPR;
  const int nvec = cols / VE;

  for (int64_t base = (int64_t)blockIdx.x * RPW; base < rows; base += (int64_t)gridDim.x * RPW) {
    const int64_t row = base + rl;
    const bool live = row < rows;
    const T* xr = x + row * ld_x;
    float v[VPT][VE];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int c = t + k * TPR;
      if (live && c < nvec) {
        Vec16<T> xv = NT ? load16_nt(xr + (int64_t)c * VE) : load16(xr + (int64_t)c * VE);
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          v[k][e] = to_f32(xv.e[e]);
          m = fmaxf(m, v[k][e]);
        }
      }
    }
    m = wave_max(m);
    if constexpr (WPR > 1) {
      if ((threadIdx.x & 63) == 0) part[rl][t / 64] = m;
      __syncthreads();
      m = part[rl][0];
#pragma unroll
      for (int i = 1; i < WPR; ++i) m = fmaxf(m, part[rl][i]);
      __syncthreads();
    }

    // exp(x - m): the max element gives exp2(0) = 1 exactly.
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int c = t + k * TPR;
      if (live && c < nvec) {
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          v[k][e] = fast_exp(v[k][e] - m);
          s += v[k][e];
        }
      }
    }
    s = wave_sum(s);
    if constexpr (WPR > 1) {
      if ((threadIdx.x & 63) == 0) part[rl][t / 64] = s;
      __syncthreads();
      s = 0.0f;
#pragma unroll
      for (int i = 0; i < WPR; ++i) s += part[rl][i];
      __syncthreads();
    }
    const float inv = 1.0f / s;

    T* yr = y + row * ld_y;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int c = t + k * TPR;
      if (live && c < nvec) {
        Vec16<T> o;
#pragma unroll
        for (int e = 0; e < VE; ++e) o.e[e] = from_f32<T>(v[k][e] * inv);
        if (NT) store16_nt(yr + (int64_t)c * VE, o);
        else store16(yr + (int64_t)c * VE, o);
      }
    }
  }
}

// Online (max, sum) state: sum is relative to max.
struct MaxSum {
  float m, s;
};

__device__ __forceinline__ MaxSum combine(MaxSum a, MaxSum b) {
  const float m = fmaxf(a.m, b.m);
  if (m == -INFINITY) return {m, 0.0f};
  const float sa = a.m == -INFINITY ? 0.0f : a.s * fast_exp(a.m - m);
  const float sb = b.m == -INFINITY ? 0.0f : b.s * fast_exp(b.m - m);
  return {m, sa + sb};
}

// Any width / alignment: a 256-thread workgroup per row (rows by grid
// stride), two passes over global memory (online max/sum, then normalise).
template <typename T>
__device__ void softmax_generic_row(const T* __restrict__ xr, T* __restrict__ yr, int cols,
                                    MaxSum* part) {
  MaxSum st{-INFINITY, 0.0f};
  for (int c = threadIdx.x; c < cols; c += 256) {
    const float v = to_f32(xr[c]);
    if (v > st.m) {
      // exp(v - v) is 1, or NaN for v = +inf, as in the reference op.
      st.s = st.s * fast_exp(st.m - v) + fast_exp(v - v);
      st.m = v;
    } else if (v != v) {
      st = {v, v};  // NaN poisons the row
    } else if (v != -INFINITY) {
      st.s += fast_exp(v - st.m);
    }
  }
  // wave-level combine through shuffles
  for (int off = 1; off < 64; off <<= 1) {
    MaxSum o{__shfl_xor(st.m, off, 64), __shfl_xor(st.s, off, 64)};
    st = (st.m != st.m || o.m != o.m) ? MaxSum{NAN, NAN} : combine(st, o);
  }
  if ((threadIdx.x & 63) == 0) part[threadIdx.x / 64] = st;
  __syncthreads();
  st = part[0];
  for (int i = 1; i < 4; ++i) {
    st = (st.m != st.m || part[i].m != part[i].m) ? MaxSum{NAN, NAN} : combine(st, part[i]);
  }
  __syncthreads();  // part is rewritten for the next row
  const float inv = 1.0f / st.s;
  for (int c = threadIdx.x; c < cols; c += 256) {
    yr[c] = from_f32<T>(fast_exp(to_f32(xr[c]) - st.m) * inv);
  }
}

template <typename T>
__global__ void __launch_bounds__(256)
softmax_generic_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t rows, int cols,
                       int64_t ld_x, int64_t ld_y) {
  __shared__ MaxSum part[4];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    softmax_generic_row(x + row * ld_x, y + row * ld_y, cols, part);
  }
}

template <typename T, int VPT, int TPR, bool NT>
void launch_vec(const T* x, T* y, int64_t rows, int cols, int64_t ld_x, int64_t ld_y,
                hipStream_t s) {
  constexpr int RPW = TPR >= 256 ? 1 : 256 / TPR;
  const unsigned grid = row_grid((rows + RPW - 1) / RPW);
  softmax_vec_kernel<T, VPT, TPR, NT><<<dim3(grid), dim3(TPR * RPW), 0, s>>>(
      x, y, rows, cols, ld_x, ld_y);
}

template <typename T>
int dispatch(const void* xv, void* yv, int64_t rows, int64_t cols, int64_t ld_x, int64_t ld_y,
             hipStream_t s) {
  const T* x = static_cast<const T*>(xv);
  T* y = static_cast<T*>(yv);
  constexpr int VE = Vec16<T>::VE;
  const bool vec_ok = cols % VE == 0 && ld_x % VE == 0 && ld_y % VE == 0 && aligned16(x) &&
                      aligned16(y);
  const int64_t nvec = cols / VE;
  const int c = (int)cols;
#define AK_LAUNCH(VPT, TPR) launch_vec<T, VPT, TPR, true>(x, y, rows, c, ld_x, ld_y, s)
  if (!vec_ok || nvec > 8192) {
    softmax_generic_kernel<T><<<dim3(row_grid(rows)), dim3(256), 0, s>>>(x, y, rows, c, ld_x, ld_y);
  } else if (nvec <= 64) AK_LAUNCH(1, 64);
  else if (nvec <= 128) AK_LAUNCH(2, 64);
  else if (nvec <= 256) AK_LAUNCH(1, 256);
  else if (nvec <= 512) AK_LAUNCH(1, 512);
  else if (nvec <= 1024) AK_LAUNCH(1, 1024);
  else if (nvec <= 2048) AK_LAUNCH(2, 1024);
  else if (nvec <= 4096) AK_LAUNCH(4, 1024);
  else AK_LAUNCH(8, 1024);
#undef AK_LAUNCH
  return ak_check_launch("ak_softmax_fwd");
}

}  // namespace
}  // namespace ak

extern "C" int ak_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols, int64_t ld_x,
                              int64_t ld_y, int dtype, void* stream) {
  const char* name = "ak_softmax_fwd";
  if (ak_dtype_size(dtype) == 0) return ak_set_error(AK_ERR_UNSUPPORTED, "%s: unsupported dtype code %d", name, dtype);
  if (rows < 0 || cols <= 0 || cols > (int64_t)1 << 30)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: bad shape rows=%lld cols=%lld", name, (long long)rows, (long long)cols);
  if (ld_x < cols || ld_y < cols) return ak_set_error(AK_ERR_INVALID_ARG, "%s: row pitch smaller than cols", name);
  if (!ak_extent_ok(rows, ld_x, cols, ak_dtype_size(dtype)) || !ak_extent_ok(rows, ld_y, cols, ak_dtype_size(dtype)))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: rows=%lld x pitch exceed 64-bit addressing", name, (long long)rows);
  if (rows == 0) return AK_OK;
  if (!x || !y) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  hipStream_t s = ak_stream(stream);
  switch (dtype) {
    case AK_DTYPE_F32: return ak::dispatch<float>(x, y, rows, cols, ld_x, ld_y, s);
    case AK_DTYPE_F16: return ak::dispatch<ak::f16>(x, y, rows, cols, ld_x, ld_y, s);
    default: return ak::dispatch<ak::bf16>(x, y, rows, cols, ld_x, ld_y, s);
  }
}
