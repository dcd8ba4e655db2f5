// Mamba-1 selective scan forward and the diagonal linear recurrence, gfx950.
//
// Mamba-1 (semantics of selective_scan_ref, external/mamba/mamba_ssm/ops/
// selective_scan_interface.py:115-181, fp32 state):
//   delta' = softplus?(delta + delta_bias)          (per channel d, step l)
//   h[n]   = exp(delta' * A[d, n]) * h[n] + delta' * u * B[g, n, l]
//   y      = sum_n h[n] * C[g, n, l] + D[d] * u
//   out    = y * silu(z)                            (silu in fp32)
//
// Work decomposition: one lane per (channel, state). A wave holds 4 channels
// x 16 states, so the recurrence over l stays sequential inside a lane and
// needs no carry between chunks (batch * dim * 16 lanes is enough parallel
// work to fill all 256 CUs for Mamba shapes). Per step and lane the VALU
// cost is one multiply for the exponent argument, one exp2 (half rate), one
// multiply for delta*u*B and one FMA for the state; delta and delta*u come
// from the lane that loaded them through DPP row_newbcast fused into those
// multiplies. The output reduction over states goes through a padded LDS
// transpose every 16 steps: lane (c, j) then owns step j of channel c and
// folds h[n] * C[n] with 16 FMAs. B and C are staged per 64-step tile in LDS
// as fp32, converted once per workgroup. exp uses exp2 with A pre-scaled by
// log2(e), like the reference kernel (selective_scan_fwd_kernel.cuh:173-177).
#include "ak_common.h"

namespace ak {
namespace {

constexpr int kScanT = 64;          // steps per LDS tile
constexpr int kScanCh = 16;         // channels per workgroup (4 waves x 4)
constexpr int kBStride = kScanT + 4; // Bs[n][l] row pitch (floats)
constexpr int kCStride = 20;        // Cs[l][n] row pitch (floats)
constexpr int kHJ = 20;             // hbuf[c][j][n] step pitch (floats)
constexpr int kHC = 16 * kHJ + 16;  // hbuf channel pitch: 336 = 16 mod 64

struct ScanParams {
  const void* u;
  const void* delta;
  const float* A;
  const void* B;
  const void* C;
  const float* D;
  const void* z;
  const float* delta_bias;
  void* out;
  float* last_state;
  int batch, dim, seqlen, dstate, ngroups, ch_per_group, tiles_per_group;
  int64_t u_bs, u_ds, d_bs, d_ds, A_ds, B_bs, B_gs, B_ns, C_bs, C_gs, C_ns, z_bs, z_ds, o_bs, o_ds;
  int softplus;
};

// Broadcast lane k of each 16-lane row (DPP row_newbcast:k).
__device__ __forceinline__ float row_bcast(float v, int k) {
  switch (k) {
    case 0: return dpp<0x150>(v);
    case 1: return dpp<0x151>(v);
    case 2: return dpp<0x152>(v);
    case 3: return dpp<0x153>(v);
    case 4: return dpp<0x154>(v);
    case 5: return dpp<0x155>(v);
    case 6: return dpp<0x156>(v);
    case 7: return dpp<0x157>(v);
    case 8: return dpp<0x158>(v);
    case 9: return dpp<0x159>(v);
    case 10: return dpp<0x15A>(v);
    case 11: return dpp<0x15B>(v);
    case 12: return dpp<0x15C>(v);
    case 13: return dpp<0x15D>(v);
    case 14: return dpp<0x15E>(v);
    default: return dpp<0x15F>(v);
  }
}

__device__ __forceinline__ float softplus_f32(float x) {
  // torch.nn.functional.softplus with beta=1, threshold=20.
  return x > 20.0f ? x : log1pf(expf(x));
}

// silu(z) = z / (1 + exp(-z)) with the hardware exp2 and reciprocal (about
// 1 ulp each), evaluated once per output element.
__device__ __forceinline__ float silu_fast(float z) {
  return z * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * kLog2e));
}

template <typename T>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  return to_f32(static_cast<const T*>(p)[i]);
}

template <typename TU, typename TD, typename TBC>
__global__ void __launch_bounds__(256)
mamba_scan_fwd_kernel(ScanParams p) {
  __shared__ float Bs[16 * kBStride];
  __shared__ float Cs[kScanT * kCStride];
  __shared__ float hbuf[4][4 * kHC];

  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int c = lane / 16;  // channel within the wave
  const int n = lane % 16;  // state owned by this lane

  const int per_batch = p.ngroups * p.tiles_per_group;
  const int b = blockIdx.x / per_batch;
  const int g = (blockIdx.x % per_batch) / p.tiles_per_group;
  const int tile = blockIdx.x % p.tiles_per_group;
  const int ch_local = tile * kScanCh + wave * 4 + c;  // channel index inside the group
  const bool ch_ok = ch_local < p.ch_per_group;
  const int d = g * p.ch_per_group + (ch_ok ? ch_local : 0);
  const bool n_ok = n < p.dstate;

  const float a_scaled = (ch_ok && n_ok) ? p.A[(int64_t)d * p.A_ds + n] * kLog2e : 0.0f;
  const float dbias = p.delta_bias ? p.delta_bias[d] : 0.0f;
  const float dskip = p.D ? p.D[d] : 0.0f;

  const int64_t u_row = (int64_t)b * p.u_bs + (int64_t)d * p.u_ds;
  const int64_t d_row = (int64_t)b * p.d_bs + (int64_t)d * p.d_ds;
  const int64_t z_row = (int64_t)b * p.z_bs + (int64_t)d * p.z_ds;
  const int64_t o_row = (int64_t)b * p.o_bs + (int64_t)d * p.o_ds;
  const int64_t B_base = (int64_t)b * p.B_bs + (int64_t)g * p.B_gs;
  const int64_t C_base = (int64_t)b * p.C_bs + (int64_t)g * p.C_gs;

  float h = 0.0f;
  float* hb = hbuf[wave];

  // Global loads for one 64-step tile, issued one tile ahead of their use so
  // that their latency hides behind the previous tile's recurrence.
  struct TileRegs {
    float bv[4], cv[4];  // B / C staging: state sn, steps 4q..4q+3
    float dv[4], uv[4];  // this lane's broadcast steps 4n..4n+3
    float uo[4], zo[4];  // output steps 16*blk + n, blk = 0..3
  };
  const int sn = tid / 16, q = tid % 16;
  auto load_tile = [&](int l0, TileRegs& r) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int l = l0 + 4 * q + k;
      const bool ok = sn < p.dstate && l < p.seqlen;
      r.bv[k] = ok ? ld<TBC>(p.B, B_base + (int64_t)sn * p.B_ns + l) : 0.0f;
      r.cv[k] = ok ? ld<TBC>(p.C, C_base + (int64_t)sn * p.C_ns + l) : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int l = l0 + 4 * n + k;
      const bool ok = ch_ok && l < p.seqlen;
      r.dv[k] = ok ? ld<TD>(p.delta, d_row + l) : 0.0f;
      r.uv[k] = ok ? ld<TU>(p.u, u_row + l) : 0.0f;
    }
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int l = l0 + 16 * blk + n;
      const bool ok = ch_ok && l < p.seqlen;
      r.uo[blk] = ok ? ld<TU>(p.u, u_row + l) : 0.0f;
      r.zo[blk] = (ok && p.z) ? ld<TU>(p.z, z_row + l) : 0.0f;
    }
  };

  TileRegs cur, nxt{};
  load_tile(0, cur);
  for (int l0 = 0; l0 < p.seqlen; l0 += kScanT) {
    __syncthreads();  // previous tile's readers of Bs / Cs are done
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      Bs[sn * kBStride + 4 * q + k] = cur.bv[k];
      Cs[(4 * q + k) * kCStride + sn] = cur.cv[k];
    }
    float dl[4], du[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const bool ok = ch_ok && l0 + 4 * n + k < p.seqlen;
      float dv = cur.dv[k] + dbias;
      if (p.softplus) dv = softplus_f32(dv);
      dl[k] = ok ? dv : 0.0f;
      du[k] = dl[k] * cur.uv[k];
    }
    if (l0 + kScanT < p.seqlen) load_tile(l0 + kScanT, nxt);
    __syncthreads();

#pragma unroll
    for (int blk = 0; blk < kScanT / 16; ++blk) {
      float hv[16];
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const int src = blk * 4 + j4;  // lane in the row that owns these 4 steps
        const float* brow = &Bs[n * kBStride + 16 * blk + 4 * j4];
        const float bvals[4] = {brow[0], brow[1], brow[2], brow[3]};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float a = __builtin_amdgcn_exp2f(row_bcast(dl[k], src) * a_scaled);
          const float x = row_bcast(du[k], src) * bvals[k];
          h = fmaf(a, h, x);
          hv[4 * j4 + k] = h;
        }
      }
      // Transpose through LDS: hbuf[c][j][n] = h at step j of this block.
#pragma unroll
      for (int j = 0; j < 16; ++j) hb[c * kHC + j * kHJ + n] = hv[j];
      __builtin_amdgcn_wave_barrier();
      // Lane (c, j=n) now reduces step j of channel c over the 16 states.
      const float* hrow = &hb[c * kHC + n * kHJ];
      const float* crow = &Cs[(16 * blk + n) * kCStride];
      float y = 0.0f;
#pragma unroll
      for (int s = 0; s < 16; ++s) y = fmaf(hrow[s], crow[s], y);
      __builtin_amdgcn_wave_barrier();
      const int l = l0 + 16 * blk + n;
      if (ch_ok && l < p.seqlen) {
        float o = fmaf(dskip, cur.uo[blk], y);
        if (p.z) o *= silu_fast(cur.zo[blk]);
        static_cast<TU*>(p.out)[o_row + l] = from_f32<TU>(o);
      }
    }
    cur = nxt;
  }
  if (p.last_state && ch_ok && n_ok) {
    p.last_state[((int64_t)b * p.dim + d) * p.dstate + n] = h;
  }
}

// Diagonal recurrence over [batch, seqlen, d_inner] fp32, one lane per
// (batch, channel); consecutive lanes read consecutive channels, so every
// step is a coalesced 256-byte row segment per wave.
__global__ void __launch_bounds__(256)
diag_scan_kernel(const float* __restrict__ dA, const float* __restrict__ dBx,
                 const float* __restrict__ C, const float* __restrict__ D,
                 const float* __restrict__ x, float* __restrict__ y, int batch, int seqlen,
                 int d_inner) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)batch * d_inner) return;
  const int b = (int)(gid / d_inner);
  const int d = (int)(gid % d_inner);
  const float dd = D[d];
  float s = 0.0f;
  int64_t idx = (int64_t)b * seqlen * d_inner + d;
  for (int t = 0; t < seqlen; ++t, idx += d_inner) {
    s = fmaf(dA[idx], s, dBx[idx]);
    y[idx] = fmaf(C[idx], s, dd * x[idx]);
  }
}

template <typename TU, typename TD, typename TBC>
void launch_scan(const ScanParams& p, hipStream_t s) {
  const int grid = p.batch * p.ngroups * p.tiles_per_group;
  mamba_scan_fwd_kernel<TU, TD, TBC><<<dim3(grid), dim3(256), 0, s>>>(p);
}

template <typename TU>
int dispatch_scan(const ScanParams& p, int u_dtype, int delta_dtype, int bc_dtype, hipStream_t s) {
  const bool d32 = delta_dtype == AK_DTYPE_F32;
  const bool bc32 = bc_dtype == AK_DTYPE_F32;
  if (!d32 && delta_dtype != u_dtype) return -1;
  if (!bc32 && bc_dtype != u_dtype) return -1;
  if (d32 && bc32) launch_scan<TU, float, float>(p, s);
  else if (d32) launch_scan<TU, float, TU>(p, s);
  else if (bc32) launch_scan<TU, TU, float>(p, s);
  else launch_scan<TU, TU, TU>(p, s);
  return 0;
}

}  // namespace
}  // namespace ak

extern "C" int ak_selective_scan_fwd(
    const void* u, const void* delta, const float* A, const void* B, const void* C,
    const float* D, const void* z, const float* delta_bias, void* out, float* last_state,
    int64_t batch, int64_t dim, int64_t seqlen, int64_t dstate, int64_t ngroups,
    int64_t u_batch_stride, int64_t u_dim_stride, int64_t delta_batch_stride,
    int64_t delta_dim_stride, int64_t A_dim_stride, int64_t B_batch_stride,
    int64_t B_group_stride, int64_t B_state_stride, int64_t C_batch_stride,
    int64_t C_group_stride, int64_t C_state_stride, int64_t z_batch_stride, int64_t z_dim_stride,
    int64_t out_batch_stride, int64_t out_dim_stride, int delta_softplus, int u_dtype,
    int delta_dtype, int bc_dtype, void* stream) {
  const char* name = "ak_selective_scan_fwd";
  if (batch < 0 || dim <= 0 || seqlen < 0 || dstate <= 0 || ngroups <= 0)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: bad shape", name);
  if (dstate > 16) return ak_set_error(AK_ERR_UNSUPPORTED, "%s: dstate=%lld > 16 is not supported", name, (long long)dstate);
  if (dim % ngroups) return ak_set_error(AK_ERR_INVALID_ARG, "%s: dim %% ngroups != 0", name);
  if (ak_dtype_size(u_dtype) == 0 || ak_dtype_size(delta_dtype) == 0 || ak_dtype_size(bc_dtype) == 0)
    return ak_set_error(AK_ERR_UNSUPPORTED, "%s: unsupported dtype", name);
  if (batch > 65535 || dim > (1 << 24) || seqlen > ((int64_t)1 << 31) - ak::kScanT)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: shape too large", name);
  if (batch == 0 || seqlen == 0) return AK_OK;
  if (!u || !delta || !A || !B || !C || !out) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  ak::ScanParams p;
  p.u = u; p.delta = delta; p.A = A; p.B = B; p.C = C; p.D = D; p.z = z;
  p.delta_bias = delta_bias; p.out = out; p.last_state = last_state;
  p.batch = (int)batch; p.dim = (int)dim; p.seqlen = (int)seqlen; p.dstate = (int)dstate;
  p.ngroups = (int)ngroups; p.ch_per_group = (int)(dim / ngroups);
  p.tiles_per_group = (p.ch_per_group + ak::kScanCh - 1) / ak::kScanCh;
  if ((int64_t)p.batch * p.ngroups * p.tiles_per_group > 0x7FFFFFFF)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: grid too large", name);
  p.u_bs = u_batch_stride; p.u_ds = u_dim_stride; p.d_bs = delta_batch_stride; p.d_ds = delta_dim_stride;
  p.A_ds = A_dim_stride; p.B_bs = B_batch_stride; p.B_gs = B_group_stride; p.B_ns = B_state_stride;
  p.C_bs = C_batch_stride; p.C_gs = C_group_stride; p.C_ns = C_state_stride;
  p.z_bs = z_batch_stride; p.z_ds = z_dim_stride; p.o_bs = out_batch_stride; p.o_ds = out_dim_stride;
  p.softplus = delta_softplus ? 1 : 0;
  hipStream_t s = ak_stream(stream);
  int rc;
  switch (u_dtype) {
    case AK_DTYPE_F32: rc = ak::dispatch_scan<float>(p, u_dtype, delta_dtype, bc_dtype, s); break;
    case AK_DTYPE_F16: rc = ak::dispatch_scan<ak::f16>(p, u_dtype, delta_dtype, bc_dtype, s); break;
    default: rc = ak::dispatch_scan<ak::bf16>(p, u_dtype, delta_dtype, bc_dtype, s); break;
  }
  if (rc) return ak_set_error(AK_ERR_UNSUPPORTED, "%s: delta and B/C must be fp32 or the dtype of u", name);
  return ak_check_launch(name);
}

extern "C" int ak_diag_scan_fwd(const float* dA, const float* dBx, const float* C, const float* D,
                                const float* x, float* y, int64_t batch, int64_t seqlen,
                                int64_t d_inner, void* stream) {
  const char* name = "ak_diag_scan_fwd";
  if (batch < 0 || seqlen < 0 || d_inner <= 0) return ak_set_error(AK_ERR_INVALID_ARG, "%s: bad shape", name);
  if (batch * d_inner > 0x7FFFFFFFll) return ak_set_error(AK_ERR_INVALID_ARG, "%s: shape too large", name);
  if (batch == 0 || seqlen == 0) return AK_OK;
  if (!dA || !dBx || !C || !D || !x || !y) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  const int64_t lanes = batch * d_inner;
  const unsigned grid = (unsigned)((lanes + 255) / 256);
  ak::diag_scan_kernel<<<dim3(grid), dim3(256), 0, ak_stream(stream)>>>(dA, dBx, C, D, x, y, (int)batch,
                                                                      (int)seqlen, (int)d_inner);
  return ak_check_launch(name);
}
