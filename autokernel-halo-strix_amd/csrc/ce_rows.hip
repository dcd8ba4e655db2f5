// Cross-entropy over materialised logits [rows, vocab] for gfx950.
//
// Semantics of kernels/ce_fused.py:122-329 (forward) and :405-488 (tiny-mode
// backward) of the reference:
//   x      = softcap > 0 ? softcap * tanh(logit / softcap) : logit
//   lse    = max + log(sum(exp(x - max)))                 (always written)
//   loss   = ignored ? 0 : lse - (1 - a) * x[t] - a * mean(x)   (a = smoothing)
//   grad_i = (p_i (1 + 2 w lse) - [i == t](1 - a) - a / V)
//            * (softcap ? 1 - tanh^2 : 1) * scale
//   (w = z-loss weight: the gradient of loss + w lse^2); ignored rows get a
//   zero gradient row.
// A 256-thread workgroup owns a row (rows by grid stride), streams it with
// 16-byte loads and keeps a per-thread online (max, sum) pair, merged across
// the workgroup with wave64 shuffles and LDS. The gradient pass re-reads the
// row (it is normally still resident in L2 / MALL). The gradient scale can
// come from device memory (scale_dev), so the mean's 1 / #counted-rows and
// the upstream gradient never need a host read. ce_count_kernel and
// ce_mean_kernel reduce the targets and per-row results in one workgroup in
// a fixed order (deterministic).
#include "ak_common.h"

namespace ak {
namespace {

constexpr int kCeThreads = 256;

struct CeParams {
  float softcap, inv_softcap, ls, ls_uniform, scale, zw2;  // zw2 = 2 * z-loss weight
  const float* scale_dev;  // optional device factor of scale
  int64_t ignore_index;
  bool use_softcap, use_ls;
};

__device__ __forceinline__ float cap(const CeParams& p, float x) {
  return p.use_softcap ? p.softcap * tanh_f32(x * p.inv_softcap) : x;
}

struct MS {
  float m, s;
};

// Merge two online (max, sum-relative-to-max) states.
__device__ __forceinline__ MS merge(MS a, MS b) {
  if (a.m != a.m || b.m != b.m) return {NAN, NAN};
  const float m = fmaxf(a.m, b.m);
  if (m == -INFINITY) return {m, 0.0f};
  float s = 0.0f;
  if (a.m != -INFINITY) s += a.s * fast_exp(a.m - m);
  if (b.m != -INFINITY) s += b.s * fast_exp(b.m - m);
  return {m, s};
}

// Workgroup-wide merge; every thread returns the row result.
__device__ MS block_merge(MS st, float& sum_x) {
  for (int off = 1; off < 64; off <<= 1) {
    MS o{__shfl_xor(st.m, off, 64), __shfl_xor(st.s, off, 64)};
    st = merge(st, o);
  }
  sum_x = wave_sum(sum_x);
  __shared__ float sm[kCeThreads / 64], ss[kCeThreads / 64], sx[kCeThreads / 64];
  const int w = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) {
    sm[w] = st.m;
    ss[w] = st.s;
    sx[w] = sum_x;
  }
  __syncthreads();
  st = {sm[0], ss[0]};
  sum_x = sx[0];
#pragma unroll
  for (int i = 1; i < kCeThreads / 64; ++i) {
    st = merge(st, MS{sm[i], ss[i]});
    sum_x += sx[i];
  }
  __syncthreads();  // sm / ss / sx are rewritten for the workgroup's next row
  return st;
}

// zf = 1 + 2 w lse folds the z-loss term into the softmax part.
template <typename T>
__device__ __forceinline__ void grad_element(const CeParams& p, float xo, float m, float inv_s,
                                             float zf, float scale, int64_t idx, int64_t tgt,
                                             float tcoeff, T& out) {
  const float x = cap(p, xo);
  float g = fast_exp(x - m) * inv_s * zf;
  if (idx == tgt) g -= tcoeff;
  if (p.use_ls) g -= p.ls_uniform;
  if (p.use_softcap) {
    const float t = x * p.inv_softcap;  // == tanh(logit / softcap)
    g *= (1.0f - t * t);
  }
  out = from_f32<T>(g * scale);
}

// Writes the gradient row: zero for ignored rows, NaN for out-of-range
// targets, otherwise the softmax gradient.
template <typename T, bool VEC>
__device__ void write_grad_row(const CeParams& p, const T* __restrict__ row, T* __restrict__ grow,
                               int64_t vocab, int64_t tgt, bool ignored, bool bad, float m,
                               float s) {
  constexpr int VE = Vec16<T>::VE;
  const float inv_s = 1.0f / s;
  const float tcoeff = p.use_ls ? 1.0f - p.ls : 1.0f;
  const float zf = p.zw2 != 0.0f ? fmaf(p.zw2, m + fast_log(s), 1.0f) : 1.0f;
  const float scale = p.scale_dev ? p.scale * p.scale_dev[0] : p.scale;
  if (VEC) {
    const int64_t nvec = vocab / VE;
    for (int64_t v = threadIdx.x; v < nvec; v += kCeThreads) {
      Vec16<T> o;
      if (ignored || bad) {
#pragma unroll
        for (int e = 0; e < VE; ++e) o.e[e] = from_f32<T>(ignored ? 0.0f : NAN);
      } else {
        Vec16<T> xv = load16(row + v * VE);
#pragma unroll
        for (int e = 0; e < VE; ++e)
          grad_element<T>(p, to_f32(xv.e[e]), m, inv_s, zf, scale, v * VE + e, tgt, tcoeff, o.e[e]);
      }
      store16(grow + v * VE, o);
    }
  } else {
    for (int64_t i = threadIdx.x; i < vocab; i += kCeThreads) {
      if (ignored || bad) {
        grow[i] = from_f32<T>(ignored ? 0.0f : NAN);
      } else {
        grad_element<T>(p, to_f32(row[i]), m, inv_s, zf, scale, i, tgt, tcoeff, grow[i]);
      }
    }
  }
}

template <typename T, bool VEC>
__device__ void ce_fwd_row(const T* __restrict__ row, int64_t b, const int64_t* __restrict__ targets,
                           float* __restrict__ losses, float* __restrict__ lse_out,
                           float* __restrict__ max_out, float* __restrict__ sum_out,
                           T* __restrict__ grow, int64_t vocab, const CeParams& p) {
  constexpr int VE = Vec16<T>::VE;
  const int64_t tgt = targets[b];
  const bool ignored = tgt == p.ignore_index;
  const bool bad = !ignored && (tgt < 0 || tgt >= vocab);

  MS st{-INFINITY, 0.0f};
  float sum_x = 0.0f;
  auto consume = [&](const float* xs, int n) {
    float vm = -INFINITY;
    for (int e = 0; e < n; ++e) vm = fmaxf(vm, xs[e]);
    if (vm > st.m) {
      st.s = st.s * fast_exp(st.m - vm);
      st.m = vm;
    }
    if (st.m != -INFINITY) {
      for (int e = 0; e < n; ++e) st.s += fast_exp(xs[e] - st.m);
    }
  };
  if (VEC) {
    const int64_t nvec = vocab / VE;
    for (int64_t v = threadIdx.x; v < nvec; v += kCeThreads) {
      Vec16<T> xv = load16(row + v * VE);
      float xs[VE];
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        xs[e] = cap(p, to_f32(xv.e[e]));
        if (p.use_ls) sum_x += xs[e];
        if (xs[e] != xs[e]) st = {NAN, NAN};
      }
      if (st.m == st.m) consume(xs, VE);
    }
  } else {
    for (int64_t i = threadIdx.x; i < vocab; i += kCeThreads) {
      float xv = cap(p, to_f32(row[i]));
      if (p.use_ls) sum_x += xv;
      if (xv != xv) st = {NAN, NAN};
      if (st.m == st.m) consume(&xv, 1);
    }
  }
  st = block_merge(st, sum_x);
  const float lse = st.m + fast_log(st.s);

  if (threadIdx.x == 0) {
    lse_out[b] = lse;
    if (max_out) max_out[b] = st.m;
    if (sum_out) sum_out[b] = st.s;
    float loss;
    if (ignored) {
      loss = 0.0f;
    } else if (bad) {
      loss = NAN;
    } else {
      const float xt = cap(p, to_f32(row[tgt]));
      loss = p.use_ls ? lse - (1.0f - p.ls) * xt - p.ls * (sum_x / (float)vocab) : lse - xt;
    }
    losses[b] = loss;
  }
  if (grow) write_grad_row<T, VEC>(p, row, grow, vocab, tgt, ignored, bad, st.m, st.s);
}

// One 256-thread workgroup per row, rows by grid stride (the loop bound is
// uniform per workgroup, so block_merge's barriers are reached by all waves).
template <typename T, bool VEC>
__global__ void __launch_bounds__(kCeThreads)
ce_fwd_kernel(const T* __restrict__ logits, const int64_t* __restrict__ targets,
              float* __restrict__ losses, float* __restrict__ lse_out,
              float* __restrict__ max_out, float* __restrict__ sum_out,
              T* __restrict__ grad, int64_t rows, int64_t vocab, int64_t ld, int64_t ld_g,
              CeParams p) {
  for (int64_t b = blockIdx.x; b < rows; b += gridDim.x)
    ce_fwd_row<T, VEC>(logits + b * ld, b, targets, losses, lse_out, max_out, sum_out,
                       grad ? grad + b * ld_g : nullptr, vocab, p);
}

template <typename T, bool VEC>
__global__ void __launch_bounds__(kCeThreads)
ce_bwd_tiny_kernel(const T* __restrict__ logits, const int64_t* __restrict__ targets,
                   const float* __restrict__ row_max, const float* __restrict__ row_sum,
                   T* __restrict__ grad, int64_t rows, int64_t vocab, int64_t ld, int64_t ld_g,
                   CeParams p) {
  for (int64_t b = blockIdx.x; b < rows; b += gridDim.x) {
    const int64_t tgt = targets[b];
    const bool ignored = tgt == p.ignore_index;
    const bool bad = !ignored && (tgt < 0 || tgt >= vocab);
    write_grad_row<T, VEC>(p, logits + b * ld, grad + b * ld_g, vocab, tgt, ignored, bad,
                           row_max[b], row_sum[b]);
  }
}

constexpr int kCeReduceThreads = 1024;

// Sum of per-thread values over one 1024-thread workgroup in a fixed order
// (wave DPP / shuffle tree, then the 16 wave sums in index order). Every
// thread returns the total.
template <typename V>
__device__ V workgroup_sum_fixed(V v, V* lds) {
  if constexpr (std::is_same<V, float>::value) {
    v = wave_sum(v);
  } else {
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  }
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x / 64] = v;
  __syncthreads();
  V t = lds[0];
  for (int i = 1; i < kCeReduceThreads / 64; ++i) t += lds[i];
  return t;
}

// denom[0] = max(1, #rows whose target is not ignore_index), denom[1] = 1 / denom[0].
__global__ void __launch_bounds__(kCeReduceThreads)
ce_count_kernel(const int64_t* __restrict__ targets, int64_t rows, int64_t ignore_index,
                float* __restrict__ denom) {
  __shared__ long long lds[kCeReduceThreads / 64];
  long long n = 0;
  for (int64_t i = threadIdx.x; i < rows; i += kCeReduceThreads) n += targets[i] != ignore_index;
  n = workgroup_sum_fixed<long long>(n, lds);
  if (threadIdx.x == 0) {
    const float d = n > 0 ? (float)n : 1.0f;
    denom[0] = d;
    denom[1] = 1.0f / d;
  }
}

// loss[0] = (sum over counted rows of losses + w * sum of lse^2) / max(1, #counted),
// per-thread partials in row order, then workgroup_sum_fixed. n_valid (nullable)
// receives the count.
__global__ void __launch_bounds__(kCeReduceThreads)
ce_mean_kernel(const float* __restrict__ losses, const float* __restrict__ lse,
               const int64_t* __restrict__ targets, int64_t rows, int64_t ignore_index,
               float zw, float* __restrict__ loss, int64_t* __restrict__ n_valid) {
  __shared__ float lds_f[kCeReduceThreads / 64];
  __shared__ long long lds_n[kCeReduceThreads / 64];
  float s = 0.0f;
  long long n = 0;
  for (int64_t i = threadIdx.x; i < rows; i += kCeReduceThreads) {
    if (targets[i] == ignore_index) continue;
    float v = losses[i];
    if (zw != 0.0f) v = fmaf(zw * lse[i], lse[i], v);
    s += v;
    ++n;
  }
  s = workgroup_sum_fixed<float>(s, lds_f);
  n = workgroup_sum_fixed<long long>(n, lds_n);
  if (threadIdx.x == 0) {
    loss[0] = s / (n > 0 ? (float)n : 1.0f);
    if (n_valid) n_valid[0] = n;
  }
}

CeParams make_params(float softcap, int64_t ignore_index, float ls, float scale, int64_t vocab,
                     float zw = 0.0f, const float* scale_dev = nullptr) {
  CeParams p;
  p.use_softcap = softcap > 0.0f;
  p.softcap = softcap;
  p.inv_softcap = p.use_softcap ? 1.0f / softcap : 0.0f;
  p.use_ls = ls > 0.0f;
  p.ls = ls;
  p.ls_uniform = ls / (float)vocab;
  p.scale = scale;
  p.zw2 = 2.0f * zw;
  p.scale_dev = scale_dev;
  p.ignore_index = ignore_index;
  return p;
}

// Rows are walked by grid stride and indexed in 64 bits; the one limit is
// that the last row's end must be addressable.
int check(const void* logits, const int64_t* targets, void* grad, int64_t rows, int64_t vocab,
          int64_t ld, int64_t ld_g, int dtype, const char* name) {
  if (ak_dtype_size(dtype) == 0) return ak_set_error(AK_ERR_UNSUPPORTED, "%s: unsupported dtype code %d", name, dtype);
  if (rows < 0 || vocab <= 0) return ak_set_error(AK_ERR_INVALID_ARG, "%s: bad shape rows=%lld vocab=%lld", name, (long long)rows, (long long)vocab);
  if (ld < vocab || (grad && ld_g < vocab)) return ak_set_error(AK_ERR_INVALID_ARG, "%s: row pitch smaller than vocab", name);
  if (!ak_extent_ok(rows, ld, vocab, ak_dtype_size(dtype)) ||
      (grad && !ak_extent_ok(rows, ld_g, vocab, ak_dtype_size(dtype))))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: rows=%lld x pitch exceed 64-bit addressing", name, (long long)rows);
  if (rows > 0 && (!logits || !targets)) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  return AK_OK;
}

template <typename T>
bool vec_ok(const void* logits, const void* grad, int64_t vocab, int64_t ld, int64_t ld_g) {
  constexpr int VE = Vec16<T>::VE;
  bool ok = vocab % VE == 0 && ld % VE == 0 && aligned16(logits);
  if (grad) ok = ok && ld_g % VE == 0 && aligned16(grad);
  return ok;
}

template <typename T>
void launch_fwd(const void* logits, const int64_t* targets, float* losses, float* lse, float* mx,
                float* sm, void* grad, int64_t rows, int64_t vocab, int64_t ld, int64_t ld_g,
                const CeParams& p, hipStream_t s) {
  const T* lg = static_cast<const T*>(logits);
  T* g = static_cast<T*>(grad);
  const dim3 grid(row_grid(rows)), block(kCeThreads);
  if (vec_ok<T>(logits, grad, vocab, ld, ld_g))
    ce_fwd_kernel<T, true><<<grid, block, 0, s>>>(lg, targets, losses, lse, mx, sm, g, rows, vocab, ld, ld_g, p);
  else
    ce_fwd_kernel<T, false><<<grid, block, 0, s>>>(lg, targets, losses, lse, mx, sm, g, rows, vocab, ld, ld_g, p);
}

template <typename T>
void launch_bwd(const void* logits, const int64_t* targets, const float* mx, const float* sm,
                void* grad, int64_t rows, int64_t vocab, int64_t ld, int64_t ld_g,
                const CeParams& p, hipStream_t s) {
  const T* lg = static_cast<const T*>(logits);
  T* g = static_cast<T*>(grad);
  const dim3 grid(row_grid(rows)), block(kCeThreads);
  if (vec_ok<T>(logits, grad, vocab, ld, ld_g))
    ce_bwd_tiny_kernel<T, true><<<grid, block, 0, s>>>(lg, targets, mx, sm, g, rows, vocab, ld, ld_g, p);
  else
    ce_bwd_tiny_kernel<T, false><<<grid, block, 0, s>>>(lg, targets, mx, sm, g, rows, vocab, ld, ld_g, p);
}

}  // namespace
}  // namespace ak

extern "C" int ak_ce_fwd(const void* logits, const int64_t* targets, float* losses, float* lse,
                         float* row_max, float* row_sum, void* grad_logits, int64_t rows,
                         int64_t vocab, int64_t ld_logits, int64_t ld_grad, float softcap,
                         int64_t ignore_index, float label_smoothing, float scale_grad,
                         float z_loss_weight, const float* scale_dev, int dtype, void* stream) {
  const char* name = "ak_ce_fwd";
  int rc = ak::check(logits, targets, grad_logits, rows, vocab, ld_logits, ld_grad, dtype, name);
  if (rc) return rc;
  if (!(z_loss_weight >= 0.0f)) return ak_set_error(AK_ERR_INVALID_ARG, "%s: z_loss_weight must be >= 0", name);
  if (rows > 0 && (!losses || !lse)) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null losses/lse", name);
  if (rows == 0) return AK_OK;
  const ak::CeParams p = ak::make_params(softcap, ignore_index, label_smoothing, scale_grad, vocab,
                                         z_loss_weight, scale_dev);
  hipStream_t s = ak_stream(stream);
  switch (dtype) {
    case AK_DTYPE_F32: ak::launch_fwd<float>(logits, targets, losses, lse, row_max, row_sum, grad_logits, rows, vocab, ld_logits, ld_grad, p, s); break;
    case AK_DTYPE_F16: ak::launch_fwd<ak::f16>(logits, targets, losses, lse, row_max, row_sum, grad_logits, rows, vocab, ld_logits, ld_grad, p, s); break;
    default: ak::launch_fwd<ak::bf16>(logits, targets, losses, lse, row_max, row_sum, grad_logits, rows, vocab, ld_logits, ld_grad, p, s); break;
  }
  return ak_check_launch(name);
}

extern "C" int ak_ce_bwd_tiny(const void* logits, const int64_t* targets, const float* row_max,
                              const float* row_sum, void* grad_logits, int64_t rows, int64_t vocab,
                              int64_t ld_logits, int64_t ld_grad, float softcap,
                              int64_t ignore_index, float label_smoothing, float scale_grad,
                              float z_loss_weight, const float* scale_dev, int dtype,
                              void* stream) {
  const char* name = "ak_ce_bwd_tiny";
  int rc = ak::check(logits, targets, grad_logits, rows, vocab, ld_logits, ld_grad, dtype, name);
  if (rc) return rc;
  if (!(z_loss_weight >= 0.0f)) return ak_set_error(AK_ERR_INVALID_ARG, "%s: z_loss_weight must be >= 0", name);
  if (rows > 0 && (!row_max || !row_sum || !grad_logits)) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  if (rows == 0) return AK_OK;
  const ak::CeParams p = ak::make_params(softcap, ignore_index, label_smoothing, scale_grad, vocab,
                                         z_loss_weight, scale_dev);
  hipStream_t s = ak_stream(stream);
  switch (dtype) {
    case AK_DTYPE_F32: ak::launch_bwd<float>(logits, targets, row_max, row_sum, grad_logits, rows, vocab, ld_logits, ld_grad, p, s); break;
    case AK_DTYPE_F16: ak::launch_bwd<ak::f16>(logits, targets, row_max, row_sum, grad_logits, rows, vocab, ld_logits, ld_grad, p, s); break;
    default: ak::launch_bwd<ak::bf16>(logits, targets, row_max, row_sum, grad_logits, rows, vocab, ld_logits, ld_grad, p, s); break;
  }
  return ak_check_launch(name);
}

extern "C" int ak_ce_count_valid(const int64_t* targets, int64_t rows, int64_t ignore_index,
                                 float* denom, void* stream) {
  const char* name = "ak_ce_count_valid";
  if (rows < 0) return ak_set_error(AK_ERR_INVALID_ARG, "%s: rows < 0", name);
  if (!denom || (rows > 0 && !targets)) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  ak::ce_count_kernel<<<dim3(1), dim3(ak::kCeReduceThreads), 0, ak_stream(stream)>>>(
      targets, rows, ignore_index, denom);
  return ak_check_launch(name);
}

extern "C" int ak_ce_mean(const float* losses, const float* lse, const int64_t* targets,
                          int64_t rows, int64_t ignore_index, float z_loss_weight, float* loss,
                          int64_t* n_valid, void* stream) {
  const char* name = "ak_ce_mean";
  if (rows < 0) return ak_set_error(AK_ERR_INVALID_ARG, "%s: rows < 0", name);
  if (!(z_loss_weight >= 0.0f)) return ak_set_error(AK_ERR_INVALID_ARG, "%s: z_loss_weight must be >= 0", name);
  if (!loss || (rows > 0 && (!losses || !targets || (z_loss_weight > 0.0f && !lse))))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  ak::ce_mean_kernel<<<dim3(1), dim3(ak::kCeReduceThreads), 0, ak_stream(stream)>>>(
      losses, lse, targets, rows, ignore_index, z_loss_weight, loss, n_valid);
  return ak_check_launch(name);
}
