// Definitions shared by the Mamba-1 selective-scan translation units
// (selective_scan.hip: the dstate <= 16 kernels and the C-ABI entry points;
// selective_scan_wide.hip: the general kernels for dstate <= 256 and
// input-independent B / C): the parameter block, the lane-broadcast
// arithmetic and the workspace layout of the backward.
#pragma once

#include "ak_common.h"

namespace ak {

constexpr int kScanT = 64;          // steps per LDS tile
constexpr int kScanCh = 16;         // channels per workgroup (4 waves x 4)
constexpr int kBStride = kScanT + 4; // Bs[n][l] row pitch (floats)
constexpr int kCStride = 20;        // Cs[l][n] row pitch (floats)
constexpr int kHJ = 20;             // hbuf[c][j][n] step pitch (floats)
constexpr int kHC = 16 * kHJ + 16;  // hbuf channel pitch: 336 = 16 mod 64
constexpr int kCk = 16;             // steps between the states saved for the backward
constexpr int kXChunk = 2048;       // steps per chunk-state entry (the reference's chunk)

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
  void* out_prez;              // optional: y + D u before the gate (strides of out)
  float* chunk_states;         // optional: [batch, dim, xchunks, dstate, 2] (decay product, state)
  int xchunks;                 // 2048-step chunks of chunk_states
  int batch, dim, seqlen, dstate, ngroups, ch_per_group, tiles_per_group;
  int64_t u_bs, u_ds, d_bs, d_ds, A_ds, B_bs, B_gs, B_ns, C_bs, C_gs, C_ns, z_bs, z_ds, o_bs, o_ds;
  int softplus;
  // backward only (the preparation pass and the reverse pass)
  const void* dout;            // [batch, dim, seqlen], element type of u, strides go_bs / go_ds
  void* dz;                    // [batch, dim, seqlen], strides of out
  void* du;                    // [batch, dim, seqlen], strides of out
  void* ddelta;                // [batch, dim, seqlen] in delta's type, strides of out
  float* ck;                   // [batch, nchunks, dim, dstate] states before each 16-step block
                               // (the forward writes them when non-null)
  float* dB_part;              // [tiles, batch, ngroups, dstate, seqlen]
  float* dC_part;              // [tiles, batch, ngroups, dstate, seqlen]
  float* dA_part;              // [batch, dim, dstate]
  float* dD_part;              // [batch, dim]
  float* dbias_part;           // [batch, dim]
  int64_t go_bs, go_ds;
  int nchunks;
  // input-independent B / C ([dim, dstate] fp32, the reference's
  // !is_variable_B / !is_variable_C): flag, channel stride (B_ns / C_ns stay
  // the state strides), and in the backward the per-batch partial sums
  // [batch, dim, dstate] of their gradients
  int b_const, c_const;
  int64_t B_ds, C_ds;
  float* dBc_part;
  float* dCc_part;
};

// v * m, with v taken from lane K of each 16-lane row (DPP row_newbcast:K
// fused into the multiply). The DPP source must not have been written by a
// VALU instruction in the two preceding cycles; callers write it once per
// tile and separate that write from the first use with an s_nop 1.
template <int K>
__device__ __forceinline__ float mul_bcast(float v, float m) {
  float r;
  asm("v_mul_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
               : "=v"(r)
               : "v"(v), "v"(m), "i"(K));
  return r;
}

// torch.nn.functional.softplus with beta=1, threshold=20: x above 20, else
// log1p(e^x). e^x and log2 come from the hardware (about 1 ulp each);
// log1p(t) = log(1 + t) * t / ((1 + t) - 1) corrects the rounding of 1 + t
// (D. Goldberg, "What every computer scientist should know about
// floating-point arithmetic", 1991, Theorem 4), so small results keep their
// relative accuracy. About 8 instructions instead of a library log1p / exp.
__device__ __forceinline__ float softplus_f32(float x) {
  const float t = __builtin_amdgcn_exp2f(fminf(x, 20.0f) * kLog2e);
  const float u = 1.0f + t;
  const float lp = u == 1.0f ? t : __builtin_amdgcn_logf(u) * kLn2 * (t * __builtin_amdgcn_rcpf(u - 1.0f));
  return x > 20.0f ? x : lp;
}

// silu(z) = z / (1 + exp(-z)) with the hardware exp2 and reciprocal (about
// 1 ulp each), evaluated once per output element.
__device__ __forceinline__ float silu_fast(float z) {
  return z * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * kLog2e));
}


constexpr int kTJ = 36;             // tbuf[c][j][n] step pitch: float pairs, b128 reads conflict-free
constexpr int kTC = 16 * kTJ + 16;  // tbuf channel pitch: 592 = 16 mod 64 (1.5% faster than 576 or 608)
constexpr int kWP = 33;             // wbuf[lane][pair] lane pitch

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// a + b over lanes i and i ^ 32 for x, and the same for y, with x's sums
// landing in lanes 0..31 and y's in lanes 32..63.
__device__ __forceinline__ float swap32_sum(float x, float y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Row pairs (0, 1) and (2, 3): x's sums land in rows 0 and 2, y's in rows 1 and 3.
__device__ __forceinline__ float swap16_sum(float x, float y) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// acc + v * m, v from lane K of each 16-lane row (DPP as in mul_bcast).
template <int K>
__device__ __forceinline__ float fma_bcast(float v, float m, float acc) {
  asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
      : "+v"(acc)
      : "v"(v), "v"(m), "i"(K));
  return acc;
}

__device__ __forceinline__ float sigmoid_f32(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}


// Workspace of the Mamba-1 backward, each region 256-byte aligned: the states
// before every 16-step block, the per-channel-tile partial rows of a
// variable dB / dC, the per-batch partials of dA / dD / ddelta_bias and of a
// constant dB / dC.
struct ScanBwdWs {
  size_t ck, partB, partC, dA, dD, dBc, dCc, total;
};

inline ScanBwdWs scan_bwd_ws(int64_t batch, int64_t dim, int64_t seqlen, int64_t dstate,
                             int64_t ngroups, int bc_flags) {
  auto a256 = [](int64_t v) { return (size_t)((v + 255) & ~(int64_t)255); };
  const int64_t tiles = (dim / ngroups + kScanCh - 1) / kScanCh;
  const int64_t nck = (seqlen + kCk - 1) / kCk;
  const bool bc = bc_flags & AK_SCAN_B_CONST, cc = bc_flags & AK_SCAN_C_CONST;
  ScanBwdWs w;
  w.ck = a256(batch * nck * dim * dstate * 4);
  w.partB = bc ? 0 : a256(tiles * batch * ngroups * dstate * seqlen * 4);
  w.partC = cc ? 0 : a256(tiles * batch * ngroups * dstate * seqlen * 4);
  w.dA = a256(batch * dim * dstate * 4);
  w.dD = a256(batch * dim * 4);
  w.dBc = bc ? a256(batch * dim * dstate * 4) : 0;
  w.dCc = cc ? a256(batch * dim * dstate * 4) : 0;
  w.total = w.ck + w.partB + w.partC + w.dA + 2 * w.dD + w.dBc + w.dCc;
  return w;
}

// Complex-A scan (selective_scan_complex.hip). Workspace of its backward,
// each region 256-byte aligned: the complex states every 16 steps and the
// pre-gate output (used when the caller gives no saved states), the
// per-4-channel-tile partial rows of a variable dB / dC, the per-batch
// partials of dA / dD / ddelta_bias and of a constant dB / dC.
struct ZWs {
  size_t ck, prez, partB, partC, dA, dD, dBc, dCc, total;
};
ZWs scan_complex_bwd_ws(int64_t batch, int64_t dim, int64_t seqlen, int64_t dstate, int64_t ngroups,
                        int bc_flags);
// The forward writes out / out_prez / last_state / chunk_states / checkpoints
// (complex where the real forward writes fp32). The backward restarts from
// p.ck / p.out_prez when saved, else re-runs the forward into the workspace,
// and writes every gradient. Both return nonzero for unsupported dtypes.
int launch_scan_complex_fwd(ScanParams p, int u_dtype, int delta_dtype, int bc_dtype, hipStream_t s);
int launch_scan_complex_bwd(ScanParams p, const ZWs& ws, void* workspace, bool saved, int u_dtype,
                            int delta_dtype, int bc_dtype, void* dB, void* dC, float* dA, float* dD,
                            float* ddelta_bias, hipStream_t s);
// Zero-step complex backward: dA, dD, ddelta_bias and a constant dB / dC are
// sums over nothing.
void launch_scan_complex_zero(int dim, int dstate, float* dA, float* dD, float* ddelta_bias,
                              float* dBc, float* dCc, hipStream_t s);

// Whether the general kernels (selective_scan_wide.hip) take the call:
// more than 16 states, or an input-independent B or C.
inline bool scan_needs_wide(const ScanParams& p) {
  return p.dstate > 16 || p.b_const || p.c_const;
}

// Launchers of the general kernels (selective_scan_wide.hip). The forward
// writes out / out_prez / last_state / chunk_states / checkpoints as
// ak_selective_scan_fwd describes; with prep it is instead the backward's
// preparation pass (checkpoints and dz). The reverse pass fills the
// workspace partials that scan_bwd_finish sums.
int launch_scan_wide_fwd(const ScanParams& p, bool prep, int u_dtype, int delta_dtype,
                         int bc_dtype, hipStream_t s);
int launch_scan_wide_bwd(const ScanParams& p, int u_dtype, int delta_dtype, int bc_dtype,
                         hipStream_t s);
// The whole-tile reverse pass (selective_scan_bwd_fast.hip): launches it and
// returns true when the shape and layout qualify, else launches nothing. It
// may take 32 channels per workgroup, and then sets p.tiles_per_group to the
// number of dB / dC partial rows it wrote per group (the sums that follow
// read that many).
bool launch_scan_bwd_fast(ScanParams& p, int u_dtype, int delta_dtype, int bc_dtype,
                          hipStream_t s);

}  // namespace ak
