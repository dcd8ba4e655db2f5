// RMSNorm backward and fused residual-add + RMSNorm backward for gfx950.
//
// Per row, in fp32 (x is the forward input, or the saved hidden state
// x + residual of the fused forward):
//   r  = 1 / sqrt(mean(x^2) + eps)
//   n  = x * r                              the normalised row
//   g  = dy * w
//   dx = r * (g - n * sum(g * n) / cols)    (+ d_hidden in the fused form)
//   dw = sum over rows of dy * n            (fp32)
// the gradient computed by the reference's HIP backward kernels
// (kernels/hip/rmsnorm_backward.py:60-189, kernels/hip/
// fused_residual_rmsnorm_backward.py:61-197), rounded once to the element
// type.
//
// Work decomposition. As in the forward kernel, TPR threads own a row with
// one or more 16-byte vectors each, and they keep the same columns for every
// row their workgroup visits, so the weight gradient of those columns
// accumulates in registers. A workgroup walks rows with a grid stride and
// loads the next row's vectors before it reduces the current one. The two row
// sums (sum x^2 and sum g*x; sum g*n = r * sum g*x) share one reduction
// (DPP within a wave, double-buffered LDS across waves: one barrier per row).
// Each workgroup then writes its partial weight gradient (one fp32 row per row
// slot) into the caller's workspace and a second kernel sums the partial
// rows per column in a fixed order: dw is deterministic (the reference
// accumulated it with fp32 atomics).
#include <atomic>
#include <mutex>

#include "ak_common.h"

namespace ak {
namespace {

// workgroups of the row pass: one per CU (a sweep at the C3 shape measured
// 256 / 384 / 512 / 1024 workgroups at 94.8 / 104.4 / 97.3 / 99.9 us; fewer
// workgroups also mean fewer partial weight-gradient rows to sum)
constexpr int kBwdMaxGrid = 256;
constexpr int kBwdMaxParts = 2048; // partial dw rows (kBwdMaxGrid x at most 4 row slots)

template <typename T, bool ADD_DH, int VPT, int TPR>
__global__ void __launch_bounds__(TPR >= 256 ? TPR : 256)
rownorm_bwd_vec_kernel(const T* __restrict__ x, const T* __restrict__ w,
                       const T* __restrict__ dy, const T* __restrict__ dh, T* __restrict__ dx,
                       float* __restrict__ part, int64_t rows, int cols, int64_t ld_x,
                       int64_t ld_dy, int64_t ld_dh, int64_t ld_dx, float eps) {
  constexpr int VE = Vec16<T>::VE;
  constexpr int RPW = TPR >= 256 ? 1 : 256 / TPR;  // rows per workgroup pass
  constexpr int WPR = TPR / 64;                      // waves per row
  static_assert(TPR % 64 == 0, "rows are owned by whole waves");
  __shared__ float red[2][RPW][WPR][2];

  const int t = threadIdx.x % TPR;
  const int rl = threadIdx.x / TPR;
  const int nvec = cols / VE;

  float wf[VPT][VE], dwacc[VPT][VE];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = min(t + k * TPR, nvec - 1);
    const Vec16<T> wv = load16(w + (int64_t)v * VE);
#pragma unroll
    for (int e = 0; e < VE; ++e) {
      wf[k][e] = to_f32(wv.e[e]);
      dwacc[k][e] = 0.0f;
    }
  }

  // Raw vectors of one row. Loads are unconditional, from clamped (always
  // valid) rows and vectors; rows and vectors past the end are masked where
  // the values are used.
  struct RowRegs {
    Vec16<T> x[VPT], g[VPT], h[VPT];
  };
  auto load_row = [&](int64_t row, RowRegs& R) {
    const int64_t rc = min(row, rows - 1);
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int64_t off = (int64_t)min(t + k * TPR, nvec - 1) * VE;
      R.x[k] = load16_nt(x + rc * ld_x + off);
      R.g[k] = load16_nt(dy + rc * ld_dy + off);
      if constexpr (ADD_DH) R.h[k] = load16_nt(dh + rc * ld_dh + off);
    }
  };

  const int64_t stride = (int64_t)gridDim.x * RPW;
  RowRegs cur, nxt;
  load_row((int64_t)blockIdx.x * RPW + rl, cur);
  int par = 0;
  for (int64_t base = (int64_t)blockIdx.x * RPW; base < rows; base += stride, par ^= 1) {
    const int64_t row = base + rl;
    const bool live = row < rows;
    load_row(row + stride, nxt);

    float xf[VPT][VE], gf[VPT][VE];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const bool ok = live && t + k * TPR < nvec;
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        xf[k][e] = ok ? to_f32(cur.x[k].e[e]) : 0.0f;
        gf[k][e] = ok ? to_f32(cur.g[k].e[e]) : 0.0f;
        s1 = fmaf(xf[k][e], xf[k][e], s1);
        s2 = fmaf(gf[k][e] * wf[k][e], xf[k][e], s2);
      }
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    if constexpr (WPR > 1) {
      if ((threadIdx.x & 63) == 0) {
        red[par][rl][t / 64][0] = s1;
        red[par][rl][t / 64][1] = s2;
      }
      __syncthreads();
      s1 = 0.0f;
      s2 = 0.0f;
#pragma unroll
      for (int i = 0; i < WPR; ++i) {
        s1 += red[par][rl][i][0];
        s2 += red[par][rl][i][1];
      }
    }
    const float r = 1.0f / sqrtf(s1 / (float)cols + eps);
    const float cg = r * s2 / (float)cols;  // sum(g * n) / cols

#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = t + k * TPR;
      Vec16<T> out;
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        const float nrm = xf[k][e] * r;
        float d = r * (gf[k][e] * wf[k][e] - nrm * cg);
        if constexpr (ADD_DH) d += to_f32(cur.h[k].e[e]);
        out.e[e] = from_f32<T>(d);
        dwacc[k][e] = fmaf(gf[k][e], nrm, dwacc[k][e]);
      }
      if (live && v < nvec) store16_nt(dx + row * ld_dx + (int64_t)v * VE, out);
    }
    cur = nxt;
  }

  if (part != nullptr) {
    float* prow = part + (int64_t)(blockIdx.x * RPW + rl) * cols;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = t + k * TPR;
      if (v < nvec) {
#pragma unroll
        for (int e = 0; e < VE; e += 4) {
          const u32x4 q = {__builtin_bit_cast(uint32_t, dwacc[k][e]),
                           __builtin_bit_cast(uint32_t, dwacc[k][e + 1]),
                           __builtin_bit_cast(uint32_t, dwacc[k][e + 2]),
                           __builtin_bit_cast(uint32_t, dwacc[k][e + 3])};
          *reinterpret_cast<u32x4*>(prow + (int64_t)v * VE + e) = q;
        }
      }
    }
  }
}

// Any width or alignment: 256 threads per row with scalar accesses. The row
// is read twice (sums, then gradients); the workgroup's partial dw row lives
// in the workspace and is updated by the thread that owns each column.
template <typename T, bool ADD_DH>
__global__ void __launch_bounds__(256)
rownorm_bwd_generic_kernel(const T* __restrict__ x, const T* __restrict__ w,
                           const T* __restrict__ dy, const T* __restrict__ dh,
                           T* __restrict__ dx, float* __restrict__ part, int64_t rows, int cols,
                           int64_t ld_x, int64_t ld_dy, int64_t ld_dh, int64_t ld_dx, float eps) {
  __shared__ float red[2][4][2];
  float* prow = part ? part + (int64_t)blockIdx.x * cols : nullptr;
  if (prow)
    for (int c = threadIdx.x; c < cols; c += 256) prow[c] = 0.0f;
  int par = 0;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x, par ^= 1) {
    float s1 = 0.0f, s2 = 0.0f;
    for (int c = threadIdx.x; c < cols; c += 256) {
      const float xv = to_f32(x[row * ld_x + c]);
      const float g = to_f32(dy[row * ld_dy + c]) * to_f32(w[c]);
      s1 = fmaf(xv, xv, s1);
      s2 = fmaf(g, xv, s2);
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    if ((threadIdx.x & 63) == 0) {
      red[par][threadIdx.x / 64][0] = s1;
      red[par][threadIdx.x / 64][1] = s2;
    }
    __syncthreads();
    s1 = (red[par][0][0] + red[par][1][0]) + (red[par][2][0] + red[par][3][0]);
    s2 = (red[par][0][1] + red[par][1][1]) + (red[par][2][1] + red[par][3][1]);
    const float r = 1.0f / sqrtf(s1 / (float)cols + eps);
    const float cg = r * s2 / (float)cols;
    for (int c = threadIdx.x; c < cols; c += 256) {
      const float xv = to_f32(x[row * ld_x + c]);
      const float dyv = to_f32(dy[row * ld_dy + c]);
      const float nrm = xv * r;
      float d = r * (dyv * to_f32(w[c]) - nrm * cg);
      if constexpr (ADD_DH) d += to_f32(dh[row * ld_dh + c]);
      dx[row * ld_dx + c] = from_f32<T>(d);
      if (prow) prow[c] = fmaf(dyv, nrm, prow[c]);
    }
  }
}

// dw[c] = sum over the partial rows p of part[p][c], in a fixed order: a
// 1024-thread workgroup owns 64 columns; wave q (of 16) sums the rows
// p = q + 16 i, 32 rows per pass with all 32 loads issued before the first
// add (the partial rows come back from beyond L2, so the pass is one round
// trip), folded pairwise; the 16 wave sums are then added in wave order.
constexpr int kColWaves = 16;
constexpr int kColBatch = 32;
__global__ void __launch_bounds__(64 * kColWaves)
colsum_kernel(const float* __restrict__ part, float* __restrict__ dw, int nparts, int cols) {
  __shared__ float acc[kColWaves][64];
  const int cl = threadIdx.x % 64, q = threadIdx.x / 64;
  const int c = blockIdx.x * 64 + cl;
  const int cc = min(c, cols - 1);
  float tot = 0.0f;
  for (int p0 = q; p0 < nparts; p0 += kColBatch * kColWaves) {
    float a[kColBatch];
#pragma unroll
    for (int i = 0; i < kColBatch; ++i) {
      const int p = min(p0 + i * kColWaves, nparts - 1);
      a[i] = part[(int64_t)p * cols + cc];
    }
#pragma unroll
    for (int i = 0; i < kColBatch; ++i)
      if (p0 + i * kColWaves >= nparts) a[i] = 0.0f;
#pragma unroll
    for (int w = kColBatch / 2; w > 0; w /= 2)
#pragma unroll
      for (int i = 0; i < w; ++i) a[i] += a[i + w];
    tot += a[0];
  }
  acc[q][cl] = tot;
  __syncthreads();
  if (q == 0 && c < cols) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kColWaves; ++i) s += acc[i][cl];
    dw[c] = s;
  }
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

size_t bwd_ws_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  const int64_t parts = rows + 3 < kBwdMaxParts ? rows + 3 : kBwdMaxParts;
  return align256((size_t)parts * (size_t)cols * sizeof(float));
}

// Launch plan of the backward's row pass: the kernel (the generic one, or a
// vector kernel with VPT vectors per thread and TPR threads per row), its
// grid, and the number of partial weight-gradient rows it writes (one per
// workgroup row slot), which colsum_kernel then sums.
struct BwdPlan {
  bool generic;
  int vpt, tpr, grid, nparts;
};

template <typename T>
BwdPlan plan_bwd(const void* x, const void* w, const void* dy, const void* dh, const void* dx,
                 int64_t rows, int64_t cols, int64_t ld_x, int64_t ld_dy, int64_t ld_dh,
                 int64_t ld_dx) {
  constexpr int VE = Vec16<T>::VE;
  bool vec_ok = cols % VE == 0 && ld_x % VE == 0 && ld_dy % VE == 0 && ld_dx % VE == 0 &&
                aligned16(x) && aligned16(w) && aligned16(dy) && aligned16(dx);
  if (dh) vec_ok = vec_ok && ld_dh % VE == 0 && aligned16(dh);
  const int64_t nvec = cols / VE;
  BwdPlan p{};
  if (!vec_ok || nvec > 8192) {
    p.generic = true;
    p.grid = (int)(rows < kBwdMaxGrid ? rows : kBwdMaxGrid);
    p.nparts = p.grid;
    return p;
  }
  p.vpt = nvec <= 1024 ? 1 : nvec <= 2048 ? 2 : nvec <= 4096 ? 4 : 8;
  p.tpr = nvec <= 64 ? 64 : nvec <= 128 ? 128 : nvec <= 256 ? 256 : nvec <= 512 ? 512 : 1024;
  const int rpw = p.tpr >= 256 ? 1 : 256 / p.tpr;
  const int64_t blocks = (rows + rpw - 1) / rpw;
  p.grid = (int)(blocks < kBwdMaxGrid ? blocks : kBwdMaxGrid);
  p.nparts = p.grid * rpw;
  return p;
}

// Bytes of partial weight-gradient rows a plan writes.
size_t plan_ws_bytes(const BwdPlan& p, int64_t cols) {
  return align256((size_t)p.nparts * (size_t)cols * sizeof(float));
}

template <typename T, bool ADD_DH>
void run_bwd(const BwdPlan& plan, const void* xv, const void* wv, const void* dyv,
             const void* dhv, void* dxv, float* dw, float* part, int64_t rows, int64_t cols,
             int64_t ld_x, int64_t ld_dy, int64_t ld_dh, int64_t ld_dx, float eps,
             hipStream_t s) {
  const T* x = static_cast<const T*>(xv);
  const T* w = static_cast<const T*>(wv);
  const T* dy = static_cast<const T*>(dyv);
  const T* dh = static_cast<const T*>(dhv);
  T* dx = static_cast<T*>(dxv);
  if (!dw) part = nullptr;
  const int c = (int)cols;
  const dim3 grid(plan.grid);
#define AK_VEC(VPT, TPR)                                                                       \
  rownorm_bwd_vec_kernel<T, ADD_DH, VPT, TPR><<<grid, dim3(TPR >= 256 ? TPR : 256), 0, s>>>( \
      x, w, dy, dh, dx, part, rows, c, ld_x, ld_dy, ld_dh, ld_dx, eps)
  if (plan.generic) {
    rownorm_bwd_generic_kernel<T, ADD_DH><<<grid, dim3(256), 0, s>>>(
        x, w, dy, dh, dx, part, rows, c, ld_x, ld_dy, ld_dh, ld_dx, eps);
  } else if (plan.tpr == 64) AK_VEC(1, 64);
  else if (plan.tpr == 128) AK_VEC(1, 128);
  else if (plan.tpr == 256) AK_VEC(1, 256);
  else if (plan.tpr == 512) AK_VEC(1, 512);
  else if (plan.vpt == 1) AK_VEC(1, 1024);
  else if (plan.vpt == 2) AK_VEC(2, 1024);
  else if (plan.vpt == 4) AK_VEC(4, 1024);
  else AK_VEC(8, 1024);
#undef AK_VEC
  if (dw) colsum_kernel<<<dim3((c + 63) / 64), dim3(64 * kColWaves), 0, s>>>(part, dw, plan.nparts, c);
}

BwdPlan plan_for(const void* x, const void* w, const void* dy, const void* dh, const void* dx,
                 int64_t rows, int64_t cols, int64_t ld_x, int64_t ld_dy, int64_t ld_dh,
                 int64_t ld_dx, int dtype) {
  switch (dtype) {
    case AK_DTYPE_F32: return plan_bwd<float>(x, w, dy, dh, dx, rows, cols, ld_x, ld_dy, ld_dh, ld_dx);
    case AK_DTYPE_F16: return plan_bwd<f16>(x, w, dy, dh, dx, rows, cols, ld_x, ld_dy, ld_dh, ld_dx);
    default: return plan_bwd<bf16>(x, w, dy, dh, dx, rows, cols, ld_x, ld_dy, ld_dh, ld_dx);
  }
}

// Argument checks shared by the entry points (no HIP call).
int check_bwd_args(const char* name, int64_t rows, int64_t cols, int64_t ld_x, int64_t ld_dy,
                   int64_t ld_dh, int64_t ld_dx, bool has_dh, int dtype) {
  if (ak_dtype_size(dtype) == 0)
    return ak_set_error(AK_ERR_UNSUPPORTED, "%s: unsupported dtype code %d", name, dtype);
  if (rows < 0 || cols <= 0 || cols > (int64_t)1 << 30)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: bad shape rows=%lld cols=%lld", name,
                        (long long)rows, (long long)cols);
  if (ld_x < cols || ld_dy < cols || ld_dx < cols || (has_dh && ld_dh < cols))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: row pitch smaller than cols", name);
  const int esz = ak_dtype_size(dtype);
  if (!ak_extent_ok(rows, ld_x, cols, esz) || !ak_extent_ok(rows, ld_dy, cols, esz) ||
      !ak_extent_ok(rows, ld_dx, cols, esz) || (has_dh && !ak_extent_ok(rows, ld_dh, cols, esz)))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: rows=%lld x pitch exceed 64-bit addressing", name,
                        (long long)rows);
  return AK_OK;
}

// Enqueues the backward with the partial rows in `part` (checked by the caller).
int enqueue_bwd(const char* name, const BwdPlan& plan, const void* x, const void* w,
                const void* dy, const void* dh, void* dx, float* dw, float* part, int64_t rows,
                int64_t cols, int64_t ld_x, int64_t ld_dy, int64_t ld_dh, int64_t ld_dx,
                float eps, int dtype, hipStream_t s) {
  if (rows == 0) {
    // no rows: dw is all zeros (a fixed-order sum over no partial rows)
    if (dw) colsum_kernel<<<dim3((unsigned)((cols + 63) / 64)), dim3(64 * kColWaves), 0, s>>>(nullptr, dw, 0, (int)cols);
    return ak_check_launch(name);
  }
#define AK_BWD(TT)                                                                              \
  (dh ? run_bwd<TT, true>(plan, x, w, dy, dh, dx, dw, part, rows, cols, ld_x, ld_dy, ld_dh, ld_dx, eps, s) \
      : run_bwd<TT, false>(plan, x, w, dy, dh, dx, dw, part, rows, cols, ld_x, ld_dy, ld_dh, ld_dx, eps, s))
  switch (dtype) {
    case AK_DTYPE_F32: AK_BWD(float); break;
    case AK_DTYPE_F16: AK_BWD(f16); break;
    default: AK_BWD(bf16); break;
  }
#undef AK_BWD
  return ak_check_launch(name);
}

int bwd_entry(const char* name, const void* x, const void* w, const void* dy, const void* dh,
              void* dx, float* dw, void* ws, size_t ws_bytes, int64_t rows, int64_t cols,
              int64_t ld_x, int64_t ld_dy, int64_t ld_dh, int64_t ld_dx, float eps, int dtype,
              void* stream) {
  int rc = check_bwd_args(name, rows, cols, ld_x, ld_dy, ld_dh, ld_dx, dh != nullptr, dtype);
  if (rc) return rc;
  if (rows > 0 && (!x || !w || !dy || !dx))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  if (dw && rows > 0) {
    if (!ws || !aligned16(ws))
      return ak_set_error(AK_ERR_INVALID_ARG, "%s: workspace must be non-null and 16-byte aligned", name);
    if (ws_bytes < bwd_ws_bytes(rows, cols))
      return ak_set_error(AK_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu", name,
                          ws_bytes, bwd_ws_bytes(rows, cols));
  }
  const BwdPlan plan = plan_for(x, w, dy, dh, dx, rows, cols, ld_x, ld_dy, ld_dh, ld_dx, dtype);
  return enqueue_bwd(name, plan, x, w, dy, dh, dx, dw, static_cast<float*>(ws), rows, cols, ld_x,
                     ld_dy, ld_dh, ld_dx, eps, dtype, ak_stream(stream));
}

// ---------------------------------------------------------------------------
// Scratch of the no-allocation entry point: the partial weight-gradient rows
// live in this file-scope device array (one copy per GPU, held until the
// process ends) instead of a caller workspace. The array is cut into
// kNoAllocSlots slots of kNoAllocSlotBytes, and each stream that calls the
// entry point on a device gets a slot of its own (the first kNoAllocSlots
// streams, for the life of the process): work queued on different streams,
// such as a captured graph replayed beside eager calls, never shares partial
// rows, and calls on one stream are ordered by the stream. In host code the
// array's name is only a stand-in; its device address is queried once per
// device with hipGetSymbolAddress (with that device current) and kept in
// g_scratch_addr.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocSlotBytes = (size_t)16 << 20;  // 16 MiB per stream
constexpr int kNoAllocSlots = 4;
constexpr int kMaxDevices = 64;

__device__ __align__(256) float scratch[kNoAllocSlots * kNoAllocSlotBytes / sizeof(float)];

std::atomic<float*> g_scratch_addr[kMaxDevices];

// Per device: the streams that own the slots, in slot order.
struct SlotTable {
  std::mutex m;
  hipStream_t owner[kNoAllocSlots];
  int used = 0;
};
SlotTable g_slots[kMaxDevices];

// Device address of `scratch` on the current device (queried on first use),
// and the device's index.
int scratch_addr(const char* name, float** out, int* dev_out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0)
    return ak_set_error(AK_ERR_LAUNCH, "%s: no current HIP device", name);
  if (dev >= kMaxDevices)
    return ak_set_error(AK_ERR_UNSUPPORTED, "%s: device %d >= %d", name, dev, kMaxDevices);
  float* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!p) {
    void* addr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !addr)
      return ak_set_error(AK_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed: %s", name,
                          hipGetErrorString(e));
    p = static_cast<float*>(addr);
    g_scratch_addr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  *dev_out = dev;
  return AK_OK;
}

// The slot of `stream` on device `dev`, assigning a free one on the stream's
// first call; more than kNoAllocSlots streams on one device are refused.
int scratch_slot(const char* name, int dev, hipStream_t stream, int* slot) {
  SlotTable& t = g_slots[dev];
  std::lock_guard<std::mutex> lock(t.m);
  for (int i = 0; i < t.used; ++i)
    if (t.owner[i] == stream) {
      *slot = i;
      return AK_OK;
    }
  if (t.used == kNoAllocSlots)
    return ak_set_error(AK_ERR_UNSUPPORTED,
                        "%s: the fixed scratch has %d per-stream slots on device %d and %d "
                        "streams already own them; call from one of those streams or use "
                        "ak_fused_add_rmsnorm_bwd with a workspace",
                        name, kNoAllocSlots, dev, kNoAllocSlots);
  t.owner[t.used] = stream;
  *slot = t.used++;
  return AK_OK;
}

}  // namespace
}  // namespace ak

extern "C" size_t ak_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols) {
  return ak::bwd_ws_bytes(rows, cols);
}

extern "C" int ak_rmsnorm_bwd(const void* x, const void* weight, const void* grad_out,
                              void* grad_x, float* grad_weight, void* workspace,
                              size_t workspace_bytes, int64_t rows, int64_t cols, int64_t ld_x,
                              int64_t ld_g, int64_t ld_gx, float eps, int dtype, void* stream) {
  return ak::bwd_entry("ak_rmsnorm_bwd", x, weight, grad_out, nullptr, grad_x, grad_weight,
                       workspace, workspace_bytes, rows, cols, ld_x, ld_g, 0, ld_gx, eps, dtype,
                       stream);
}

extern "C" int ak_fused_add_rmsnorm_bwd(const void* hidden, const void* weight,
                                        const void* grad_hidden, const void* grad_normed,
                                        void* grad_x, float* grad_weight, void* workspace,
                                        size_t workspace_bytes, int64_t rows, int64_t cols,
                                        int64_t ld_h, int64_t ld_gh, int64_t ld_gn,
                                        int64_t ld_gx, float eps, int dtype, void* stream) {
  return ak::bwd_entry("ak_fused_add_rmsnorm_bwd", hidden, weight, grad_normed, grad_hidden,
                       grad_x, grad_weight, workspace, workspace_bytes, rows, cols, ld_h, ld_gn,
                       ld_gh, ld_gx, eps, dtype, stream);
}

extern "C" int ak_fused_add_rmsnorm_bwd_noalloc(const void* hidden, const void* weight,
                                                const void* grad_hidden, const void* grad_normed,
                                                void* grad_x, float* grad_weight, int64_t rows,
                                                int64_t cols, int64_t ld_h, int64_t ld_gh,
                                                int64_t ld_gn, int64_t ld_gx, float eps,
                                                int dtype, void* stream) {
  const char* name = "ak_fused_add_rmsnorm_bwd_noalloc";
  int rc = ak::check_bwd_args(name, rows, cols, ld_h, ld_gn, ld_gh, ld_gx, grad_hidden != nullptr,
                              dtype);
  if (rc) return rc;
  const ak::BwdPlan plan = ak::plan_for(hidden, weight, grad_normed, grad_hidden, grad_x,
                                              rows, cols, ld_h, ld_gn, ld_gh, ld_gx, dtype);
  const size_t need = grad_weight && rows > 0 ? ak::plan_ws_bytes(plan, cols) : 0;
  if (need > ak::kNoAllocSlotBytes)
    return ak_set_error(AK_ERR_WORKSPACE,
                        "%s: %zu bytes of scratch needed (%d partial rows x %lld cols x 4), "
                        "a stream's slot of the fixed scratch holds %zu; use "
                        "ak_fused_add_rmsnorm_bwd with a workspace",
                        name, need, plan.nparts, (long long)cols, ak::kNoAllocSlotBytes);
  if (rows > 0 && (!hidden || !weight || !grad_normed || !grad_x))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  const hipStream_t s = ak_stream(stream);
  float* part = nullptr;
  if (need > 0) {
    int dev = -1, slot = -1;
    rc = ak::scratch_addr(name, &part, &dev);
    if (rc) return rc;
    rc = ak::scratch_slot(name, dev, s, &slot);
    if (rc) return rc;
    part += (size_t)slot * (ak::kNoAllocSlotBytes / sizeof(float));
  }
  return ak::enqueue_bwd(name, plan, hidden, weight, grad_normed, grad_hidden, grad_x,
                         grad_weight, part, rows, cols, ld_h, ld_gn, ld_gh, ld_gx, eps, dtype, s);
}
