// Mamba-1 selective scan, general kernels (gfx950): any dstate up to 256 and
// input-independent B / C, forward and backward. The dstate <= 16 path with
// variable B / C (every Mamba-1 model's default) runs the specialised
// kernels of selective_scan.hip; these take everything else the reference
// binding accepts (selective_scan.cpp:262: dstate <= 256; :115-121,
// selective_scan_interface.py:138-160: B / C of shape [dim, dstate]).
//
// Lane layout as in the specialised kernels: a wave holds 4 channels x 16
// lanes, a workgroup 16 channels. Lane n of a channel owns the state slots
// s = n + 16 i, i < KS = ceil(dstate / 16). Tiles are 16 steps, one state
// checkpoint block. Per tile, lane n holds delta' and delta' u of step n;
// every other lane of its 16-lane row takes them with DPP row_newbcast fused
// into its multiplies, as in the specialised kernels. The slot loop is a run-
// time loop whose per-slot state (h; in the backward the state gradient g,
// the dA sum, the checkpointed state, A) lives in LDS, each entry read and
// written only by its owning lane, so one kernel serves every dstate without
// register arrays sized by dstate. Per slot and tile a lane runs the 16-step
// recurrence and adds h * C into 16 per-step partial outputs; the 16 lanes'
// partials of a step are summed through a per-wave LDS transpose. Variable
// B / C of the tile are staged in LDS as fp32 (rows 16 floats + 4 pad:
// the 16 lanes' b128 row reads hit disjoint banks); constant B / C are read
// once per workgroup into the same space, [channel][state].
//
// Backward (reverse over tiles, as mamba_scan_bwd_kernel): per slot the
// tile's decays and states are recomputed from the checkpoint, then the
// state gradient runs backwards; the per-step sums over states of g B and
// A a h_{l-1} (du, ddelta) go through the LDS transpose; dB / dC of a
// variable B / C are summed over the wave's 4 channels with the permlane
// pair reduction and over the 4 waves in LDS for 4 slots at a time, one
// partial row per channel tile, summed in a fixed order by the finish pass;
// a constant B / C accumulates per lane over steps and per batch in the
// workspace. Every gradient is bitwise reproducible.
#include "scan_common.h"

namespace ak {
namespace {

constexpr int kWT = 16;        // steps per tile (= kCk)
constexpr int kWBP = 20;       // staged B / C row pitch (floats)
constexpr int kYJ = 17;        // transpose buffer step pitch (scalar reads conflict-free)
constexpr int kYC = 16 * kYJ;  // transpose buffer channel pitch
constexpr int kYW = 4 * kYC;   // transpose buffer per wave
constexpr int kWbW = 64 * kWP; // dB / dC pair-sum buffer per wave

// Per-step sum over the 16 lanes of a row of v[j] (j = 0..15, one value per
// step): lane (c, n) returns the sum for step n. Through a per-wave LDS
// transpose; buf holds this wave's kYW floats.
__device__ __forceinline__ float row_transpose_sum(const float (&v)[16], float* buf, int c, int n) {
#pragma unroll
  for (int j = 0; j < 16; ++j) buf[c * kYC + j * kYJ + n] = v[j];
  __builtin_amdgcn_wave_barrier();
  float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int k = 0; k < 16; ++k) s4[k & 3] += buf[c * kYC + n * kYJ + k];
  __builtin_amdgcn_wave_barrier();
  return (s4[0] + s4[1]) + (s4[2] + s4[3]);
}

// Dynamic LDS layout (float offsets).
struct WideLayout {
  int bs, cs, hk, hs, as, gs, da, dbc, dcc, x, total;
};

__host__ __device__ constexpr WideLayout wide_layout(int ks, int dstate, bool bc, bool cc, bool bwd) {
  WideLayout L{};
  const int stage = ks * 16 * kWBP;               // variable: 16 ks rows x kWBP
  const int konst = kScanCh * dstate;             // constant: [channel][state]
  const int per_slot = ks * 256;
  int o = 0;
  L.bs = o; o += bc ? konst : stage;
  L.cs = o; o += cc ? konst : stage;
  if (!bwd) {
    L.hs = o; o += per_slot;
    L.as = o; o += per_slot;
    L.x = o; o += 4 * kYW;
  } else {
    L.hk = o; o += per_slot;   // checkpointed state at the tile start
    L.gs = o; o += per_slot;   // state gradient
    L.da = o; o += per_slot;   // dA sum
    L.as = o; o += per_slot;   // A (natural)
    L.dbc = o; o += bc ? per_slot : 0;
    L.dcc = o; o += cc ? per_slot : 0;
    L.x = o; o += (bc && cc) ? 4 * kYW : (4 * kWbW > 4 * kYW ? 4 * kWbW : 4 * kYW);
  }
  L.total = o;
  return L;
}

// Tile loads, issued a tile ahead from clamped (always valid) addresses in
// storage type; masking and conversion at the use.
template <typename TU, typename TD, typename TBC, int KSMAX, bool kBwd>
struct WideRegs {
  TBC bv[KSMAX], cv[KSMAX];  // staging rows s = tid / 16 + 16 k, step tid % 16
  TD dv;                     // this lane's step l0 + n
  TU uv, zv, gv;             // u, z, dout at l0 + n
  TU yv;                     // backward: the forward's pre-gate output at l0 + n
  float ckv[kBwd ? KSMAX : 1];  // backward: checkpointed state of slot k at the tile start
};

template <typename TU, typename TD, typename TBC, int KSMAX, bool kPrep>
__global__ void __launch_bounds__(256)
mamba_scan_wide_fwd_kernel(ScanParams p, int ks) {
  extern __shared__ float lds[];
  const int tid = threadIdx.x;
  const int wave = tid / 64, lane = tid % 64;
  const int c = lane / 16, n = lane % 16;
  const int wc = wave * 4 + c;

  const int per_batch = p.ngroups * p.tiles_per_group;
  const int b = blockIdx.x / per_batch;
  const int g = (blockIdx.x % per_batch) / p.tiles_per_group;
  const int tile = blockIdx.x % p.tiles_per_group;
  const int ch_local = tile * kScanCh + wc;
  const bool ch_ok = ch_local < p.ch_per_group;
  const int d = g * p.ch_per_group + (ch_ok ? ch_local : 0);
  const int d0 = g * p.ch_per_group + tile * kScanCh;  // the workgroup's first channel

  const WideLayout Lo = wide_layout(ks, p.dstate, p.b_const, p.c_const, false);
  float* Bs = lds + Lo.bs;
  float* Cs = lds + Lo.cs;
  float* Hs = lds + Lo.hs;
  float* As = lds + Lo.as;
  float* yb = lds + Lo.x + wave * kYW;

  const float dbias = p.delta_bias ? p.delta_bias[d] : 0.0f;
  const float dskip = p.D ? p.D[d] : 0.0f;
  // per-slot state and A (log2 e scaled); constant B / C of the workgroup's
  // channels: [channel][state], channels past the group's end read as 0
  for (int i = 0; i < ks; ++i) {
    const int s = n + 16 * i;
    const bool ok = ch_ok && s < p.dstate;
    Hs[i * 256 + tid] = 0.0f;
    As[i * 256 + tid] = ok ? p.A[(int64_t)d * p.A_ds + s] * kLog2e : 0.0f;
  }
  if (p.b_const || p.c_const) {
    for (int e = tid; e < kScanCh * p.dstate; e += 256) {
      const int ch = e / p.dstate, s = e % p.dstate;
      const bool ok = tile * kScanCh + ch < p.ch_per_group;
      const int64_t dd = d0 + (ok ? ch : 0);
      if (p.b_const) Bs[e] = ok ? static_cast<const float*>(p.B)[dd * p.B_ds + (int64_t)s * p.B_ns] : 0.0f;
      if (p.c_const) Cs[e] = ok ? static_cast<const float*>(p.C)[dd * p.C_ds + (int64_t)s * p.C_ns] : 0.0f;
    }
  }

  const int64_t u_row = (int64_t)b * p.u_bs + (int64_t)d * p.u_ds;
  const int64_t d_row = (int64_t)b * p.d_bs + (int64_t)d * p.d_ds;
  const int64_t z_row = (int64_t)b * p.z_bs + (int64_t)d * p.z_ds;
  const int64_t o_row = (int64_t)b * p.o_bs + (int64_t)d * p.o_ds;
  const int64_t go_row = (int64_t)b * p.go_bs + (int64_t)d * p.go_ds;
  const int64_t B_base = (int64_t)b * p.B_bs + (int64_t)g * p.B_gs;
  const int64_t C_base = (int64_t)b * p.C_bs + (int64_t)g * p.C_gs;
  const TU* const zsrc = static_cast<const TU*>(p.z ? p.z : p.u);
  const int64_t zrow = p.z ? z_row : u_row;
  const int sq = tid % 16;       // staging step
  const int last_l = p.seqlen - 1;

  using Regs = WideRegs<TU, TD, TBC, KSMAX, false>;
  auto load = [&](int l0, Regs& r) {
#pragma unroll
    for (int k = 0; k < KSMAX; ++k) {
      const int s = min(tid / 16 + 16 * k, p.dstate - 1);
      const int l = min(l0 + sq, last_l);
      if (!p.b_const) r.bv[k] = static_cast<const TBC*>(p.B)[B_base + (int64_t)s * p.B_ns + l];
      if (!p.c_const) r.cv[k] = static_cast<const TBC*>(p.C)[C_base + (int64_t)s * p.C_ns + l];
    }
    const int l = min(l0 + n, last_l);
    r.dv = static_cast<const TD*>(p.delta)[d_row + l];
    r.uv = static_cast<const TU*>(p.u)[u_row + l];
    r.zv = zsrc[zrow + l];
    if constexpr (kPrep) r.gv = static_cast<const TU*>(p.dout)[go_row + l];
  };

  float dsum = 0.0f;  // sum of delta' since step 0 (chunk states)
  Regs cur, nxt{};
  load(0, cur);
  for (int l0 = 0; l0 < p.seqlen; l0 += kWT) {
    __syncthreads();  // the previous tile's readers of the staging are done
#pragma unroll
    for (int k = 0; k < KSMAX; ++k) {
      if (k < ks) {
        const int s = tid / 16 + 16 * k;
        const bool ok = s < p.dstate && l0 + sq < p.seqlen;
        if (!p.b_const) Bs[s * kWBP + sq] = ok ? to_f32(cur.bv[k]) : 0.0f;
        if (!p.c_const) Cs[s * kWBP + sq] = ok ? to_f32(cur.cv[k]) : 0.0f;
      }
    }
    const bool step_ok = ch_ok && l0 + n < p.seqlen;
    float dl = to_f32(cur.dv) + dbias;
    if (p.softplus) dl = softplus_f32(dl);
    dl = step_ok ? dl : 0.0f;
    float du = dl * to_f32(cur.uv);
    // wait states between the VALU writes of dl / du and their DPP reads
    asm volatile("s_nop 1" : "+v"(dl), "+v"(du));
    if (l0 + kWT < p.seqlen) load(l0 + kWT, nxt);
    asm volatile("" ::: "memory");
    __syncthreads();

    const int chunk = l0 / kWT;
    float yp[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) yp[j] = 0.0f;
    for (int i = 0; i < ks; ++i) {
      const int s = n + 16 * i;
      const float a2 = As[i * 256 + tid];
      float h = Hs[i * 256 + tid];
      if ((kPrep || p.ck) && ch_ok && s < p.dstate)
        p.ck[(((int64_t)b * p.nchunks + chunk) * p.dim + d) * p.dstate + s] = h;
      float bt[16], ct[16];
      if (p.b_const) {
        const float bk = Bs[wc * p.dstate + min(s, p.dstate - 1)] * (s < p.dstate ? 1.0f : 0.0f);
#pragma unroll
        for (int j = 0; j < 16; ++j) bt[j] = bk;
      } else {
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          const float4 v = *reinterpret_cast<const float4*>(&Bs[s * kWBP + 4 * j4]);
          bt[4 * j4] = v.x; bt[4 * j4 + 1] = v.y; bt[4 * j4 + 2] = v.z; bt[4 * j4 + 3] = v.w;
        }
      }
      if (p.c_const) {
        const float ck = Cs[wc * p.dstate + min(s, p.dstate - 1)] * (s < p.dstate ? 1.0f : 0.0f);
#pragma unroll
        for (int j = 0; j < 16; ++j) ct[j] = ck;
      } else {
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          const float4 v = *reinterpret_cast<const float4*>(&Cs[s * kWBP + 4 * j4]);
          ct[4 * j4] = v.x; ct[4 * j4 + 1] = v.y; ct[4 * j4 + 2] = v.z; ct[4 * j4 + 3] = v.w;
        }
      }
      float av[16], xv[16];
      static_for<0, 16>([&](auto j_c) {
        constexpr int J = decltype(j_c)::value;
        av[J] = mul_bcast<J>(dl, a2);
        xv[J] = mul_bcast<J>(du, bt[J]);
      });
#pragma unroll
      for (int j = 0; j < 16; ++j) av[j] = __builtin_amdgcn_exp2f(av[j]);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        h = fmaf(av[j], h, xv[j]);
        yp[j] = fmaf(h, ct[j], yp[j]);
      }
      Hs[i * 256 + tid] = h;
    }

    // output of step l0 + n: sum of the 16 lanes' partials
    const float y = row_transpose_sum(yp, yb, c, n);
    if (step_ok) {
      const float uv = to_f32(cur.uv);
      float o = fmaf(dskip, uv, y);
      if constexpr (kPrep) {
        if (p.z) {
          const float zv = to_f32(cur.zv);
          const float sg = sigmoid_f32(zv);
          static_cast<TU*>(p.dz)[o_row + l0 + n] =
              from_f32<TU>(to_f32(cur.gv) * o * sg * fmaf(zv, 1.0f - sg, 1.0f));
        }
      } else {
        if (p.out_prez) static_cast<TU*>(p.out_prez)[o_row + l0 + n] = from_f32<TU>(o);
        if (p.z) o *= silu_fast(to_f32(cur.zv));
        static_cast<TU*>(p.out)[o_row + l0 + n] = from_f32<TU>(o);
      }
    }
    if (!kPrep && p.chunk_states) {
      dsum += row16_sum(dl);
      const int l1 = l0 + kWT;
      if ((l1 % kXChunk == 0 || l1 >= p.seqlen) && ch_ok) {
        for (int i = 0; i < ks; ++i) {
          const int s = n + 16 * i;
          if (s >= p.dstate) break;
          float* xs = p.chunk_states +
                      ((((int64_t)b * p.dim + d) * p.xchunks + (l1 - 1) / kXChunk) * p.dstate + s) * 2;
          xs[0] = __builtin_amdgcn_exp2f(As[i * 256 + tid] * dsum);
          xs[1] = Hs[i * 256 + tid];
        }
      }
    }
    cur = nxt;
  }
  if (!kPrep && p.last_state && ch_ok) {
    for (int i = 0; i < ks; ++i) {
      const int s = n + 16 * i;
      if (s < p.dstate) p.last_state[((int64_t)b * p.dim + d) * p.dstate + s] = Hs[i * 256 + tid];
    }
  }
}

template <typename TU, typename TD, typename TBC, int KSMAX>
__global__ void __launch_bounds__(256)
mamba_scan_wide_bwd_kernel(ScanParams p, int ks) {
  extern __shared__ float lds[];
  const int tid = threadIdx.x;
  const int wave = tid / 64, lane = tid % 64;
  const int c = lane / 16, n = lane % 16;
  const int wc = wave * 4 + c;

  const int per_batch = p.ngroups * p.tiles_per_group;
  const int b = blockIdx.x / per_batch;
  const int g = (blockIdx.x % per_batch) / p.tiles_per_group;
  const int tile = blockIdx.x % p.tiles_per_group;
  const int ch_local = tile * kScanCh + wc;
  const bool ch_ok = ch_local < p.ch_per_group;
  const int d = g * p.ch_per_group + (ch_ok ? ch_local : 0);
  const int d0 = g * p.ch_per_group + tile * kScanCh;
  const bool var_bc = !p.b_const || !p.c_const;

  const WideLayout Lo = wide_layout(ks, p.dstate, p.b_const, p.c_const, true);
  float* Bs = lds + Lo.bs;
  float* Cs = lds + Lo.cs;
  float* Hk = lds + Lo.hk;
  float* Gs = lds + Lo.gs;
  float* DA = lds + Lo.da;
  float* An = lds + Lo.as;
  float* DBc = lds + Lo.dbc;
  float* DCc = lds + Lo.dcc;
  float* wb = lds + Lo.x + wave * kWbW;   // dB / dC pair sums (variable B / C)
  float* tb = lds + Lo.x + wave * kYW;    // per-step transposes (same space, later in the tile)

  const float dbias = p.delta_bias ? p.delta_bias[d] : 0.0f;
  const float dskip = p.D ? p.D[d] : 0.0f;
  for (int i = 0; i < ks; ++i) {
    const int s = n + 16 * i;
    const bool ok = ch_ok && s < p.dstate;
    Gs[i * 256 + tid] = 0.0f;
    DA[i * 256 + tid] = 0.0f;
    An[i * 256 + tid] = ok ? p.A[(int64_t)d * p.A_ds + s] : 0.0f;
    if (p.b_const) DBc[i * 256 + tid] = 0.0f;
    if (p.c_const) DCc[i * 256 + tid] = 0.0f;
  }
  if (p.b_const || p.c_const) {
    for (int e = tid; e < kScanCh * p.dstate; e += 256) {
      const int ch = e / p.dstate, s = e % p.dstate;
      const bool ok = tile * kScanCh + ch < p.ch_per_group;
      const int64_t dd = d0 + (ok ? ch : 0);
      if (p.b_const) Bs[e] = ok ? static_cast<const float*>(p.B)[dd * p.B_ds + (int64_t)s * p.B_ns] : 0.0f;
      if (p.c_const) Cs[e] = ok ? static_cast<const float*>(p.C)[dd * p.C_ds + (int64_t)s * p.C_ns] : 0.0f;
    }
  }

  const int64_t u_row = (int64_t)b * p.u_bs + (int64_t)d * p.u_ds;
  const int64_t d_row = (int64_t)b * p.d_bs + (int64_t)d * p.d_ds;
  const int64_t z_row = (int64_t)b * p.z_bs + (int64_t)d * p.z_ds;
  const int64_t o_row = (int64_t)b * p.o_bs + (int64_t)d * p.o_ds;
  const int64_t go_row = (int64_t)b * p.go_bs + (int64_t)d * p.go_ds;
  const int64_t B_base = (int64_t)b * p.B_bs + (int64_t)g * p.B_gs;
  const int64_t C_base = (int64_t)b * p.C_bs + (int64_t)g * p.C_gs;
  const TU* const zsrc = static_cast<const TU*>(p.z ? p.z : p.u);
  const int64_t zrow = p.z ? z_row : u_row;
  const TU* const ysrc = static_cast<const TU*>(p.out_prez ? p.out_prez : p.u);
  const int64_t yrow = p.out_prez ? o_row : u_row;
  const int sq = tid % 16;
  const int last_l = p.seqlen - 1;

  using Regs = WideRegs<TU, TD, TBC, KSMAX, true>;
  auto load = [&](int l0, Regs& r) {
#pragma unroll
    for (int k = 0; k < KSMAX; ++k) {
      const int s = min(tid / 16 + 16 * k, p.dstate - 1);
      const int l = min(l0 + sq, last_l);
      if (!p.b_const) r.bv[k] = static_cast<const TBC*>(p.B)[B_base + (int64_t)s * p.B_ns + l];
      if (!p.c_const) r.cv[k] = static_cast<const TBC*>(p.C)[C_base + (int64_t)s * p.C_ns + l];
      const int sl = min(n + 16 * k, p.dstate - 1);
      r.ckv[k] = p.ck[(((int64_t)b * p.nchunks + l0 / kWT) * p.dim + d) * p.dstate + sl];
    }
    const int l = min(l0 + n, last_l);
    r.dv = static_cast<const TD*>(p.delta)[d_row + l];
    r.uv = static_cast<const TU*>(p.u)[u_row + l];
    r.zv = zsrc[zrow + l];
    r.gv = static_cast<const TU*>(p.dout)[go_row + l];
    r.yv = ysrc[yrow + l];
  };
  // dy = dout * silu(z) (dout without a gate)
  auto gated = [&](float go, float zv) { return p.z ? go * zv * sigmoid_f32(zv) : go; };

  float dnext = 0.0f;  // delta' of the step after the tile (lane 0 of the row's), for a_{l+1}
  float dD_acc = 0.0f, dbias_acc = 0.0f;
  Regs cur, nxt{};
  const int t_last = last_l / kWT;
  load(t_last * kWT, cur);
  for (int t = t_last; t >= 0; --t) {
    const int l0 = t * kWT;
    __syncthreads();  // the previous tile's readers of the staging / wbuf are done
#pragma unroll
    for (int k = 0; k < KSMAX; ++k) {
      if (k < ks) {
        const int s = tid / 16 + 16 * k;
        const bool ok = s < p.dstate && l0 + sq < p.seqlen;
        if (!p.b_const) Bs[s * kWBP + sq] = ok ? to_f32(cur.bv[k]) : 0.0f;
        if (!p.c_const) Cs[s * kWBP + sq] = ok ? to_f32(cur.cv[k]) : 0.0f;
        Hk[k * 256 + tid] = cur.ckv[k];
      }
    }
    const bool step_ok = ch_ok && l0 + n < p.seqlen;
    float bd = to_f32(cur.dv) + dbias;
    if (p.softplus) bd = softplus_f32(bd);
    bd = step_ok ? bd : 0.0f;
    float bdu = bd * to_f32(cur.uv);
    float bdy = step_ok ? gated(to_f32(cur.gv), to_f32(cur.zv)) : 0.0f;
    asm volatile("s_nop 1" : "+v"(bd), "+v"(bdu), "+v"(bdy));
    if (t > 0) load(l0 - kWT, nxt);
    asm volatile("" ::: "memory");
    __syncthreads();

    float pgb[16], paw[16];  // per-step partial sums over this lane's slots
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      pgb[j] = 0.0f;
      paw[j] = 0.0f;
    }
    for (int i = 0; i < ks; ++i) {
      const int s = n + 16 * i;
      const bool s_ok = s < p.dstate;
      const float a_nat = An[i * 256 + tid];
      const float a2 = a_nat * kLog2e;
      float gs = Gs[i * 256 + tid];
      float dA = DA[i * 256 + tid];
      float a_next = __builtin_amdgcn_exp2f(dnext * a2);
      const float hstart = s_ok ? Hk[i * 256 + tid] : 0.0f;
      float bt[16], ct[16];
      if (p.b_const) {
        const float bk = s_ok ? Bs[wc * p.dstate + s] : 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) bt[j] = bk;
      } else {
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          const float4 v = *reinterpret_cast<const float4*>(&Bs[s * kWBP + 4 * j4]);
          bt[4 * j4] = v.x; bt[4 * j4 + 1] = v.y; bt[4 * j4 + 2] = v.z; bt[4 * j4 + 3] = v.w;
        }
      }
      if (p.c_const) {
        const float ck = s_ok ? Cs[wc * p.dstate + s] : 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) ct[j] = ck;
      } else {
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          const float4 v = *reinterpret_cast<const float4*>(&Cs[s * kWBP + 4 * j4]);
          ct[4 * j4] = v.x; ct[4 * j4 + 1] = v.y; ct[4 * j4 + 2] = v.z; ct[4 * j4 + 3] = v.w;
        }
      }
      // recompute the tile's decays and states from the checkpoint
      float as[16], hs[16], xv[16];
      static_for<0, 16>([&](auto j_c) {
        constexpr int J = decltype(j_c)::value;
        as[J] = mul_bcast<J>(bd, a2);
        xv[J] = mul_bcast<J>(bdu, bt[J]);
      });
#pragma unroll
      for (int j = 0; j < 16; ++j) as[j] = __builtin_amdgcn_exp2f(as[j]);
      float h = hstart;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        h = fmaf(as[j], h, xv[j]);
        hs[j] = h;
      }
      float sB = 0.0f, sC = 0.0f;  // constant B / C: this slot's sums over the tile's steps
      float pB = 0.0f, pC = 0.0f;
      const int grp = i & 3;
      static_for<0, 16>([&](auto i_c) {
        constexpr int J = 15 - decltype(i_c)::value;
        gs = fmaf(gs, a_next, mul_bcast<J>(bdy, ct[J]));
        a_next = as[J];
        const float hp = J > 0 ? hs[J > 0 ? J - 1 : 0] : hstart;
        const float w = gs * (as[J] * hp);
        pgb[J] = fmaf(gs, bt[J], pgb[J]);
        paw[J] = fmaf(a_nat, w, paw[J]);
        dA = fma_bcast<J>(bd, w, dA);
        const float cB = mul_bcast<J>(bdu, gs);
        const float cC = mul_bcast<J>(bdy, hs[J]);
        sB += cB;
        sC += cC;
        if (var_bc) {
          if constexpr (J % 2 == 1) {
            pB = cB;
            pC = cC;
          } else {
            // lanes 16 r + n: r = 0: dB at step J, 1: dB at J + 1, 2: dC at J, 3: dC at J + 1
            const float s_even = swap32_sum(cB, cC);
            const float s_odd = swap32_sum(pB, pC);
            wb[lane * kWP + 8 * grp + J / 2] = swap16_sum(s_even, s_odd);
          }
        }
      });
      Gs[i * 256 + tid] = gs;
      DA[i * 256 + tid] = dA;
      if (p.b_const) DBc[i * 256 + tid] += sB;
      if (p.c_const) DCc[i * 256 + tid] += sC;
      if (var_bc && (grp == 3 || i == ks - 1)) {
        // the group's dB / dC over the workgroup's 16 channels: one partial
        // row per channel tile (rows s, steps l0 .. l0 + 15)
        __syncthreads();
        const int j = tid % 16, n2 = tid / 16;
        for (int ii = 0; ii <= grp; ++ii) {
          const int s2 = n2 + 16 * (i - grp + ii);
#pragma unroll
          for (int v = 0; v < 2; ++v) {
            if (v == 0 ? p.b_const : p.c_const) continue;
            const int L = 16 * (2 * v + (j & 1)) + n2;
            const int off = L * kWP + 8 * ii + j / 2;
            const float sum = ((lds[Lo.x + off] + lds[Lo.x + kWbW + off]) +
                               lds[Lo.x + 2 * kWbW + off]) + lds[Lo.x + 3 * kWbW + off];
            if (s2 < p.dstate && l0 + j < p.seqlen) {
              float* part = v ? p.dC_part : p.dB_part;
              part[((((int64_t)tile * p.batch + b) * p.ngroups + g) * p.dstate + s2) * p.seqlen + l0 + j] = sum;
            }
          }
        }
        __syncthreads();
      }
    }

    // per step l0 + n: sums over all states of g B and A a h_{l-1}
    const float sgb = row_transpose_sum(pgb, tb, c, n);
    const float saw = row_transpose_sum(paw, tb, c, n);
    if (step_ok) {
      const int l = l0 + n;
      const float go = to_f32(cur.gv);
      float dyv = go;
      if (p.z) {
        const float zv = to_f32(cur.zv);
        const float sg = sigmoid_f32(zv);
        dyv = go * zv * sg;
        if (p.out_prez)
          static_cast<TU*>(p.dz)[o_row + l] =
              from_f32<TU>(go * to_f32(cur.yv) * sg * fmaf(zv, 1.0f - sg, 1.0f));
      }
      const float uv = to_f32(cur.uv);
      const float x = to_f32(cur.dv) + dbias;
      float dlt = x, ddl = fmaf(uv, sgb, saw);
      if (p.softplus) {
        dlt = softplus_f32(x);
        if (x <= 20.0f) ddl *= sigmoid_f32(x);
      }
      static_cast<TU*>(p.du)[o_row + l] = from_f32<TU>(fmaf(dskip, dyv, dlt * sgb));
      static_cast<TD*>(p.ddelta)[o_row + l] = from_f32<TD>(ddl);
      dD_acc = fmaf(dyv, uv, dD_acc);
      dbias_acc += ddl;
    }
    dnext = mul_bcast<0>(bd, 1.0f);
    cur = nxt;
  }
  for (int i = 0; i < ks; ++i) {
    const int s = n + 16 * i;
    if (!ch_ok || s >= p.dstate) break;
    const int64_t e = ((int64_t)b * p.dim + d) * p.dstate + s;
    p.dA_part[e] = DA[i * 256 + tid];
    if (p.b_const) p.dBc_part[e] = DBc[i * 256 + tid];
    if (p.c_const) p.dCc_part[e] = DCc[i * 256 + tid];
  }
  dD_acc = row16_sum(dD_acc);
  dbias_acc = row16_sum(dbias_acc);
  if (ch_ok && n == 0) {
    p.dD_part[(int64_t)b * p.dim + d] = dD_acc;
    p.dbias_part[(int64_t)b * p.dim + d] = dbias_acc;
  }
}

int wide_ks(int dstate) { return (dstate + 15) / 16; }

// Dynamic LDS above 64 KiB (dstate > 64) is requested explicitly from the
// runtime (gfx950 has 160 KiB per workgroup).
template <typename K>
void allow_lds(K kernel, size_t bytes) {
  if (bytes > 65536)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

template <typename TU, typename TD, typename TBC, bool kPrep>
void run_wide_fwd(const ScanParams& p, hipStream_t s) {
  const int ks = wide_ks(p.dstate);
  const size_t bytes =
      (size_t)wide_layout(ks, p.dstate, p.b_const, p.c_const, false).total * sizeof(float);
  const dim3 grid(p.batch * p.ngroups * p.tiles_per_group), block(256);
  if (ks <= 4) {
    mamba_scan_wide_fwd_kernel<TU, TD, TBC, 4, kPrep><<<grid, block, bytes, s>>>(p, ks);
  } else {
    allow_lds(mamba_scan_wide_fwd_kernel<TU, TD, TBC, 16, kPrep>, bytes);
    mamba_scan_wide_fwd_kernel<TU, TD, TBC, 16, kPrep><<<grid, block, bytes, s>>>(p, ks);
  }
}

template <typename TU, typename TD, typename TBC>
void run_wide_bwd(const ScanParams& p, hipStream_t s) {
  const int ks = wide_ks(p.dstate);
  const size_t bytes =
      (size_t)wide_layout(ks, p.dstate, p.b_const, p.c_const, true).total * sizeof(float);
  const dim3 grid(p.batch * p.ngroups * p.tiles_per_group), block(256);
  if (ks <= 4) {
    mamba_scan_wide_bwd_kernel<TU, TD, TBC, 4><<<grid, block, bytes, s>>>(p, ks);
  } else {
    allow_lds(mamba_scan_wide_bwd_kernel<TU, TD, TBC, 16>, bytes);
    mamba_scan_wide_bwd_kernel<TU, TD, TBC, 16><<<grid, block, bytes, s>>>(p, ks);
  }
}

template <typename TU, bool kPrep>
int dispatch_wide_fwd(const ScanParams& p, int u_dtype, int delta_dtype, int bc_dtype,
                      hipStream_t s) {
  const bool d32 = delta_dtype == AK_DTYPE_F32;
  const bool bc32 = bc_dtype == AK_DTYPE_F32;
  if (!d32 && delta_dtype != u_dtype) return -1;
  if (!bc32 && bc_dtype != u_dtype) return -1;
  if (d32 && bc32) run_wide_fwd<TU, float, float, kPrep>(p, s);
  else if (d32) run_wide_fwd<TU, float, TU, kPrep>(p, s);
  else if (bc32) run_wide_fwd<TU, TU, float, kPrep>(p, s);
  else run_wide_fwd<TU, TU, TU, kPrep>(p, s);
  return 0;
}

template <typename TU>
int dispatch_wide_bwd(const ScanParams& p, int u_dtype, int delta_dtype, int bc_dtype,
                      hipStream_t s) {
  const bool d32 = delta_dtype == AK_DTYPE_F32;
  const bool bc32 = bc_dtype == AK_DTYPE_F32;
  if (!d32 && delta_dtype != u_dtype) return -1;
  if (!bc32 && bc_dtype != u_dtype) return -1;
  if (d32 && bc32) run_wide_bwd<TU, float, float>(p, s);
  else if (d32) run_wide_bwd<TU, float, TU>(p, s);
  else if (bc32) run_wide_bwd<TU, TU, float>(p, s);
  else run_wide_bwd<TU, TU, TU>(p, s);
  return 0;
}

}  // namespace

// Dynamic LDS of the general kernels at dstate 256 and their lane layout
// stay within gfx950's 160 KiB per workgroup (checked here at compile time).
static_assert(wide_layout(16, 256, false, false, true).total * 4 <= 160 * 1024, "LDS");
static_assert(wide_layout(16, 256, true, true, true).total * 4 <= 160 * 1024, "LDS");
static_assert(wide_layout(16, 256, true, false, true).total * 4 <= 160 * 1024, "LDS");
static_assert(wide_layout(16, 256, false, false, false).total * 4 <= 160 * 1024, "LDS");

int launch_scan_wide_fwd(const ScanParams& p, bool prep, int u_dtype, int delta_dtype,
                         int bc_dtype, hipStream_t s) {
  switch (u_dtype) {
    case AK_DTYPE_F32:
      return prep ? dispatch_wide_fwd<float, true>(p, u_dtype, delta_dtype, bc_dtype, s)
                  : dispatch_wide_fwd<float, false>(p, u_dtype, delta_dtype, bc_dtype, s);
    case AK_DTYPE_F16:
      return prep ? dispatch_wide_fwd<f16, true>(p, u_dtype, delta_dtype, bc_dtype, s)
                  : dispatch_wide_fwd<f16, false>(p, u_dtype, delta_dtype, bc_dtype, s);
    default:
      return prep ? dispatch_wide_fwd<bf16, true>(p, u_dtype, delta_dtype, bc_dtype, s)
                  : dispatch_wide_fwd<bf16, false>(p, u_dtype, delta_dtype, bc_dtype, s);
  }
}

int launch_scan_wide_bwd(const ScanParams& p, int u_dtype, int delta_dtype, int bc_dtype,
                         hipStream_t s) {
  switch (u_dtype) {
    case AK_DTYPE_F32: return dispatch_wide_bwd<float>(p, u_dtype, delta_dtype, bc_dtype, s);
    case AK_DTYPE_F16: return dispatch_wide_bwd<f16>(p, u_dtype, delta_dtype, bc_dtype, s);
    default: return dispatch_wide_bwd<bf16>(p, u_dtype, delta_dtype, bc_dtype, s);
  }
}

}  // namespace ak
