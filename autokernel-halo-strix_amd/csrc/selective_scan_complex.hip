// Mamba-1 selective scan with complex A (the reference binding's complex64
// weights, selective_scan.cpp:236-240, :270-276; semantics of
// selective_scan_ref, selective_scan_interface.py:140-145, :173-174):
// forward, backward and the backward's fixed-order sums (gfx950).
//
// Layouts (strides in elements; a complex element is an interleaved
// (re, im) float pair):
//   A          complex [dim, dstate], state stride 1, dim stride A_ds;
//   B / C      input-dependent: real [batch, ngroups, dstate, 2 seqlen] in
//              the B / C element type, (re, im) of step l at 2 l and 2 l + 1;
//              input-independent: complex [dim, dstate] (B_ds / B_ns);
//   last_state complex [batch, dim, dstate]; chunk_states complex
//              [batch, dim, ceil(seqlen / 2048), dstate, 2] (decay product,
//              state); checkpoints complex [batch, ceil(seqlen / 16), dim,
//              dstate] (the state before every 16-step block).
//
// Per step l and state n: a = exp(delta' A) (magnitude exp2(delta' Re A
// log2 e), phase sincos(delta' Im A)), h = a h + delta' u B, and the output
// y = 2 Re sum_n h C + D u, then the gate.
//
// Work split: LPC lanes per channel, 64 / LPC channels per wave, 4 waves per
// workgroup, all of one group: LPC = 64 (one channel per wave) for dstate >
// 16, lane s owning the states s + 64 i, i < KS (dstate <= 64 KS); LPC = 16
// (four channels per wave) for dstate <= 16, one state per lane. Steps go in
// 16-step tiles: lanes 0..15 of a channel read the tile's per-channel inputs
// (one step each) into a per-channel LDS table that the channel's lanes read
// back, an input-dependent B / C tile is staged in LDS as fp32 for the
// workgroup, and the per-step sums over a channel's lanes go through a
// per-wave LDS transpose summed in a fixed order.
//
// Backward (reverse over tiles, from the 16-step checkpoints): per state the
// tile's decays and states are recomputed from the checkpoint, then the
// state gradient g (packed dL/dRe + i dL/dIm) runs backwards:
//   g_l = conj(a_{l+1}) g_{l+1} + 2 dy_l conj(C_l);
//   du_l += Re(conj(g_l) delta'_l B_l);  ddelta'_l += Re(conj(g_l) u_l B_l)
//        + Re(conj(g_l conj(h_{l-1})) A a_l);
//   dA += delta'_l conj(a_l) g_l conj(h_{l-1});  dB_l = delta'_l u_l g_l;
//   dC_l = 2 dy_l conj(h_l).
// An input-dependent dB / dC is summed over the workgroup's channels in a
// fixed order and written as one partial row per workgroup's channel tile; dA, dD,
// ddelta_bias and an input-independent dB / dC as per-batch partials. A
// finish launch adds the partials in a fixed order: every gradient is
// bitwise reproducible.
#include "scan_common.h"

namespace ak {
namespace {

constexpr int kZT = 16;    // steps per tile (= kCk, the checkpoint block)
constexpr int kZP = 34;    // staged B / C: floats per state row (16 steps x (re, im) + 2)
constexpr int kZW = 4;     // waves per workgroup

// Lanes per channel for a dstate, and channels per workgroup.
__host__ __device__ inline int zlpc(int dstate) { return dstate <= 16 ? 16 : 64; }
__host__ __device__ inline int zcpb(int dstate) { return kZW * (64 / zlpc(dstate)); }
constexpr int kZY = 16 * 64;  // per-wave transpose buffer (floats)

struct ZLayout {
  int bs, cs, tab, y, gb, gc, total;  // float offsets
};

__host__ __device__ inline ZLayout zlayout(int dstate, bool bvar, bool cvar, bool bwd) {
  ZLayout L{};
  auto a4 = [](int v) { return (v + 3) & ~3; };  // every region 16-byte aligned (b128 accesses)
  int o = 0;
  L.bs = o; o += a4(bvar ? dstate * kZP : 0);
  L.cs = o; o += a4(cvar ? dstate * kZP : 0);
  L.tab = o; o += zcpb(dstate) * kZT * 4;
  L.y = o; o += kZW * kZY;
  L.gb = o; o += (bwd && bvar) ? kZW * 64 * 32 : 0;
  L.gc = o; o += (bwd && cvar) ? kZW * 64 * 32 : 0;
  L.total = o;
  return L;
}

struct Cx {
  float r, i;
};
__device__ __forceinline__ Cx cmul(Cx a, Cx b) { return {a.r * b.r - a.i * b.i, a.r * b.i + a.i * b.r}; }
__device__ __forceinline__ Cx cconj(Cx a) { return {a.r, -a.i}; }

// sin and cos of x radians on the hardware's transcendental units
// (v_sin_f32 / v_cos_f32 take revolutions): x / 2 pi is reduced to [-1/2,
// 1/2] revolutions by subtracting its nearest integer, so the phase error
// grows with |x| (the rounding of x / 2 pi: about 6e-8 |x| radians). The
// reference builds its scan with fast math, so its __builtin_sincosf is a
// hardware approximation as well.
__device__ __forceinline__ void sincos_hw(float x, float* s, float* c) {
  float r = x * 0.15915494309189535f;  // 1 / (2 pi)
  r -= __builtin_rintf(r);
  *s = __builtin_amdgcn_sinf(r);
  *c = __builtin_amdgcn_cosf(r);
}

// exp(dl * A) for A = (ar, ai), ar pre-scaled by log2 e: the per-step decay
// factor, with the hardware phase
__device__ __forceinline__ Cx cexp_step(float dl, float ar2, float ai) {
  const float mag = __builtin_amdgcn_exp2f(dl * ar2);
  float sn, cs;
  sincos_hw(dl * ai, &sn, &cs);
  return {mag * cs, mag * sn};
}

// exp(dsum * A) for a chunk state's decay product: once per 2048-step chunk,
// where the phase dsum Im A can be large, so the accurate sincosf
__device__ __forceinline__ Cx cexp_chunk(float dsum, float ar2, float ai) {
  const float mag = __builtin_amdgcn_exp2f(dsum * ar2);
  float sn, cs;
  sincosf(dsum * ai, &sn, &cs);
  return {mag * cs, mag * sn};
}

// Stage the tile's input-dependent B or C (steps l0 .. l0 + 15) as fp32:
// dst[s * kZP + 2 j + reim]; steps past the end read 0.
template <typename TBC>
__device__ __forceinline__ void zstage(float* dst, const TBC* src, int64_t ns, int dstate, int l0,
                                       int seqlen, int tid) {
  for (int e = tid; e < dstate * 32; e += 256) {
    const int s = e >> 5, w = e & 31;
    const bool ok = l0 + (w >> 1) < seqlen;
    dst[s * kZP + w] = ok ? to_f32(src[(int64_t)s * ns + 2 * (int64_t)l0 + w]) : 0.0f;
  }
}

// Sum over a channel's LPC lanes of v[j] (one value per step j < 16): lane j
// of the channel returns the sum for step j, in a fixed order.
template <int LPC>
__device__ __forceinline__ float zlane_sum(const float (&v)[kZT], float* buf, int lane) {
#pragma unroll
  for (int j = 0; j < kZT; ++j) buf[j * 64 + lane] = v[j];
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
  const int cw = lane / LPC, sl = lane % LPC;
  float r = 0.0f;
  if (sl < kZT) {
    float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < LPC; k += 4) {
      const float4 q = *reinterpret_cast<const float4*>(&buf[sl * 64 + cw * LPC + k]);
      s4[0] += q.x;
      s4[1] += q.y;
      s4[2] += q.z;
      s4[3] += q.w;
    }
    r = (s4[0] + s4[1]) + (s4[2] + s4[3]);
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
  return r;
}

template <typename TU, typename TD, typename TBC, int KS, int LPC>
__global__ void __launch_bounds__(256) mamba_scan_complex_fwd_kernel(ScanParams p) {
  constexpr int CPW = 64 / LPC;  // channels per wave
  extern __shared__ float lds[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int cw = lane / LPC, sl = lane % LPC;  // channel within the wave, state lane
  const int per_batch = p.ngroups * p.tiles_per_group;
  const int b = blockIdx.x / per_batch;
  const int g = (blockIdx.x % per_batch) / p.tiles_per_group;
  const int tile = blockIdx.x % p.tiles_per_group;
  const int ch_local = tile * (kZW * CPW) + wave * CPW + cw;
  const bool ch_ok = ch_local < p.ch_per_group;
  const int d = g * p.ch_per_group + (ch_ok ? ch_local : p.ch_per_group - 1);
  const bool bvar = !p.b_const, cvar = !p.c_const;
  const ZLayout Lo = zlayout(p.dstate, bvar, cvar, false);
  float* Bs = lds + Lo.bs;
  float* Cs = lds + Lo.cs;
  float* tab = lds + Lo.tab + (wave * CPW + cw) * kZT * 4;
  float* yb = lds + Lo.y + wave * kZY;

  const float* Af = p.A;
  float ar2[KS], ai[KS];
  Cx x[KS], bc[KS], cc[KS];
#pragma unroll
  for (int i = 0; i < KS; ++i) {
    const int s = sl + LPC * i;
    const bool ok = s < p.dstate;
    const int64_t ea = 2 * ((int64_t)d * p.A_ds + (ok ? s : 0));
    ar2[i] = ok ? Af[ea] * kLog2e : 0.0f;
    ai[i] = ok ? Af[ea + 1] : 0.0f;
    x[i] = {0.0f, 0.0f};
    bc[i] = {0.0f, 0.0f};
    cc[i] = {0.0f, 0.0f};
    if (ok && p.b_const) {
      const float* q = static_cast<const float*>(p.B) + 2 * ((int64_t)d * p.B_ds + (int64_t)s * p.B_ns);
      bc[i] = {q[0], q[1]};
    }
    if (ok && p.c_const) {
      const float* q = static_cast<const float*>(p.C) + 2 * ((int64_t)d * p.C_ds + (int64_t)s * p.C_ns);
      cc[i] = {q[0], q[1]};
    }
  }
  const float dbias = p.delta_bias ? p.delta_bias[d] : 0.0f;
  const float dskip = p.D ? p.D[d] : 0.0f;
  const TU* up = static_cast<const TU*>(p.u) + (int64_t)b * p.u_bs + (int64_t)d * p.u_ds;
  const TD* dp = static_cast<const TD*>(p.delta) + (int64_t)b * p.d_bs + (int64_t)d * p.d_ds;
  const TU* zp = p.z ? static_cast<const TU*>(p.z) + (int64_t)b * p.z_bs + (int64_t)d * p.z_ds : nullptr;
  const int64_t orow = (int64_t)b * p.o_bs + (int64_t)d * p.o_ds;
  const TBC* bsrc = bvar ? static_cast<const TBC*>(p.B) + (int64_t)b * p.B_bs + (int64_t)g * p.B_gs : nullptr;
  const TBC* csrc = cvar ? static_cast<const TBC*>(p.C) + (int64_t)b * p.C_bs + (int64_t)g * p.C_gs : nullptr;

  float dsum = 0.0f;  // sum of delta' since step 0 (chunk states)
  const int nt = (p.seqlen + kZT - 1) / kZT;
  for (int t = 0; t < nt; ++t) {
    const int l0 = t * kZT;
    const int nst = min(kZT, p.seqlen - l0);
    if (p.ck && ch_ok) {
#pragma unroll
      for (int i = 0; i < KS; ++i) {
        const int s = sl + LPC * i;
        if (s < p.dstate) {
          float* q = p.ck + 2 * ((((int64_t)b * p.nchunks + t) * p.dim + d) * p.dstate + s);
          q[0] = x[i].r;
          q[1] = x[i].i;
        }
      }
    }
    __syncthreads();  // the previous tile's B / C readers are done
    if (bvar) zstage<TBC>(Bs, bsrc, p.B_ns, p.dstate, l0, p.seqlen, tid);
    if (cvar) zstage<TBC>(Cs, csrc, p.C_ns, p.dstate, l0, p.seqlen, tid);
    float u_l = 0.0f, z_l = 0.0f;
    if (sl < kZT) {
      const bool ok = sl < nst;
      const int l = l0 + (ok ? sl : 0);
      float dl = to_f32(dp[l]) + dbias;
      if (p.softplus) dl = softplus_f32(dl);
      u_l = to_f32(up[l]);
      z_l = zp ? to_f32(zp[l]) : 0.0f;
      dl = ok ? dl : 0.0f;
      tab[sl * 4 + 0] = dl;
      tab[sl * 4 + 1] = dl * u_l;
    }
    __syncthreads();
    float yp[kZT];
#pragma unroll
    for (int j = 0; j < kZT; ++j) {
      const float dl = tab[j * 4 + 0], du = tab[j * 4 + 1];
      dsum += dl;
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < KS; ++i) {
        const int s = sl + LPC * i;
        if (s < p.dstate) {
          const Cx a = cexp_step(dl, ar2[i], ai[i]);
          const Cx bv = bvar ? Cx{Bs[s * kZP + 2 * j], Bs[s * kZP + 2 * j + 1]} : bc[i];
          const Cx cv = cvar ? Cx{Cs[s * kZP + 2 * j], Cs[s * kZP + 2 * j + 1]} : cc[i];
          Cx h = cmul(a, x[i]);
          h.r = fmaf(du, bv.r, h.r);
          h.i = fmaf(du, bv.i, h.i);
          x[i] = h;
          acc += h.r * cv.r - h.i * cv.i;
        }
      }
      yp[j] = acc;
    }
    // chunk states at the end of every 2048-step chunk and of the sequence
    const int lend = l0 + nst;
    if (p.chunk_states && ch_ok && (lend % kXChunk == 0 || lend == p.seqlen)) {
      const int k = (lend - 1) / kXChunk;
#pragma unroll
      for (int i = 0; i < KS; ++i) {
        const int s = sl + LPC * i;
        if (s < p.dstate) {
          const Cx pr = cexp_chunk(dsum, ar2[i], ai[i]);
          float* q = p.chunk_states + 4 * ((((int64_t)b * p.dim + d) * p.xchunks + k) * p.dstate + s);
          q[0] = pr.r;
          q[1] = pr.i;
          q[2] = x[i].r;
          q[3] = x[i].i;
        }
      }
    }
    const float ysum = zlane_sum<LPC>(yp, yb, lane);
    if (sl < nst && ch_ok) {
      float o = fmaf(dskip, u_l, 2.0f * ysum);
      if (p.out_prez) static_cast<TU*>(p.out_prez)[orow + l0 + sl] = from_f32<TU>(o);
      if (zp) o *= silu_fast(z_l);
      if (p.out) static_cast<TU*>(p.out)[orow + l0 + sl] = from_f32<TU>(o);
    }
  }
  if (p.last_state && ch_ok) {
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      const int s = sl + LPC * i;
      if (s < p.dstate) {
        float* q = p.last_state + 2 * (((int64_t)b * p.dim + d) * p.dstate + s);
        q[0] = x[i].r;
        q[1] = x[i].i;
      }
    }
  }
}

// Backward partial sums (float offsets into the workspace are set up by the
// host): dA_part complex [batch, dim, dstate]; dD_part / dbias_part
// [batch, dim]; dBc_part / dCc_part complex [batch, dim, dstate];
// dB_part / dC_part [tiles, batch, ngroups, dstate, 2 seqlen].
template <typename TU, typename TD, typename TBC, int KS, int LPC>
__global__ void __launch_bounds__(256) mamba_scan_complex_bwd_kernel(ScanParams p) {
  constexpr int CPW = 64 / LPC;  // channels per wave
  extern __shared__ float lds[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int cw = lane / LPC, sl = lane % LPC;  // channel within the wave, state lane
  const int per_batch = p.ngroups * p.tiles_per_group;
  const int b = blockIdx.x / per_batch;
  const int g = (blockIdx.x % per_batch) / p.tiles_per_group;
  const int tile = blockIdx.x % p.tiles_per_group;
  const int ch_local = tile * (kZW * CPW) + wave * CPW + cw;
  const bool ch_ok = ch_local < p.ch_per_group;
  const int d = g * p.ch_per_group + (ch_ok ? ch_local : p.ch_per_group - 1);
  const bool bvar = !p.b_const, cvar = !p.c_const;
  const ZLayout Lo = zlayout(p.dstate, bvar, cvar, true);
  float* Bs = lds + Lo.bs;
  float* Cs = lds + Lo.cs;
  float* tab = lds + Lo.tab + (wave * CPW + cw) * kZT * 4;
  float* yb = lds + Lo.y + wave * kZY;
  float* gbB = lds + Lo.gb;
  float* gbC = lds + Lo.gc;

  float ar2[KS], arn[KS], ai[KS];
  Cx gs[KS], an[KS], accA[KS], accB[KS], accC[KS], bc[KS], cc[KS];
#pragma unroll
  for (int i = 0; i < KS; ++i) {
    const int s = sl + LPC * i;
    const bool ok = s < p.dstate;
    const int64_t ea = 2 * ((int64_t)d * p.A_ds + (ok ? s : 0));
    arn[i] = ok ? p.A[ea] : 0.0f;
    ar2[i] = arn[i] * kLog2e;
    ai[i] = ok ? p.A[ea + 1] : 0.0f;
    gs[i] = {0.0f, 0.0f};
    an[i] = {1.0f, 0.0f};
    accA[i] = {0.0f, 0.0f};
    accB[i] = {0.0f, 0.0f};
    accC[i] = {0.0f, 0.0f};
    bc[i] = {0.0f, 0.0f};
    cc[i] = {0.0f, 0.0f};
    if (ok && p.b_const) {
      const float* q = static_cast<const float*>(p.B) + 2 * ((int64_t)d * p.B_ds + (int64_t)s * p.B_ns);
      bc[i] = {q[0], q[1]};
    }
    if (ok && p.c_const) {
      const float* q = static_cast<const float*>(p.C) + 2 * ((int64_t)d * p.C_ds + (int64_t)s * p.C_ns);
      cc[i] = {q[0], q[1]};
    }
  }
  const float dbias = p.delta_bias ? p.delta_bias[d] : 0.0f;
  const float dskip = p.D ? p.D[d] : 0.0f;
  const TU* up = static_cast<const TU*>(p.u) + (int64_t)b * p.u_bs + (int64_t)d * p.u_ds;
  const TD* dp = static_cast<const TD*>(p.delta) + (int64_t)b * p.d_bs + (int64_t)d * p.d_ds;
  const TU* zp = p.z ? static_cast<const TU*>(p.z) + (int64_t)b * p.z_bs + (int64_t)d * p.z_ds : nullptr;
  const TU* gp = static_cast<const TU*>(p.dout) + (int64_t)b * p.go_bs + (int64_t)d * p.go_ds;
  const int64_t orow = ((int64_t)b * p.dim + d) * p.seqlen;  // du, ddelta, dz, out_prez: contiguous
  const TU* yp = static_cast<const TU*>(p.out_prez);
  const TBC* bsrc = bvar ? static_cast<const TBC*>(p.B) + (int64_t)b * p.B_bs + (int64_t)g * p.B_gs : nullptr;
  const TBC* csrc = cvar ? static_cast<const TBC*>(p.C) + (int64_t)b * p.C_bs + (int64_t)g * p.C_gs : nullptr;

  float dD_acc = 0.0f, dbias_acc = 0.0f;
  const int nt = (p.seqlen + kZT - 1) / kZT;
  for (int t = nt - 1; t >= 0; --t) {
    const int l0 = t * kZT;
    const int nst = min(kZT, p.seqlen - l0);
    __syncthreads();
    if (bvar) zstage<TBC>(Bs, bsrc, p.B_ns, p.dstate, l0, p.seqlen, tid);
    if (cvar) zstage<TBC>(Cs, csrc, p.C_ns, p.dstate, l0, p.seqlen, tid);
    float draw = 0.0f, dy = 0.0f;
    if (sl < kZT) {
      const bool ok = sl < nst;
      const int l = l0 + (ok ? sl : 0);
      draw = to_f32(dp[l]) + dbias;
      const float dl = ok ? (p.softplus ? softplus_f32(draw) : draw) : 0.0f;
      const float uu = to_f32(up[l]);
      const float go = ok ? to_f32(gp[l]) : 0.0f;
      dy = go;
      if (zp) {
        const float zv = to_f32(zp[l]);
        const float sg = sigmoid_f32(zv);
        dy = go * zv * sg;
        if (ok && ch_ok) {
          const float yv = to_f32(yp[orow + l]);
          static_cast<TU*>(p.dz)[orow + l] = from_f32<TU>(go * yv * sg * fmaf(zv, 1.0f - sg, 1.0f));
        }
      }
      dD_acc = fmaf(dy, uu, dD_acc);
      tab[sl * 4 + 0] = dl;
      tab[sl * 4 + 1] = dl * uu;
      tab[sl * 4 + 2] = uu;
      tab[sl * 4 + 3] = dy;
    }
    __syncthreads();
    float ddl_p[kZT], du_p[kZT];
#pragma unroll
    for (int j = 0; j < kZT; ++j) {
      ddl_p[j] = 0.0f;
      du_p[j] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      const int s = sl + LPC * i;
      const bool ok = s < p.dstate;
      const int sc = ok ? s : 0;
      Cx x0 = {0.0f, 0.0f};
      if (ok) {
        const float* q = p.ck + 2 * ((((int64_t)b * p.nchunks + t) * p.dim + d) * p.dstate + s);
        x0 = {q[0], q[1]};
      }
      Cx xs[kZT], as[kZT];
      Cx h = x0;
#pragma unroll
      for (int j = 0; j < kZT; ++j) {
        const float dl = tab[j * 4 + 0], dv = tab[j * 4 + 1];
        const Cx a = cexp_step(dl, ar2[i], ai[i]);
        const Cx bv = bvar ? Cx{Bs[sc * kZP + 2 * j], Bs[sc * kZP + 2 * j + 1]} : bc[i];
        Cx hn = cmul(a, h);
        hn.r = fmaf(dv, bv.r, hn.r);
        hn.i = fmaf(dv, bv.i, hn.i);
        h = hn;
        xs[j] = h;
        as[j] = a;
      }
      Cx gg = gs[i], anx = an[i], dAa = accA[i], dBa = accB[i], dCa = accC[i];
      float gB[2 * kZT], gC[2 * kZT];
#pragma unroll
      for (int j = kZT - 1; j >= 0; --j) {
        const float dl = tab[j * 4 + 0], dv = tab[j * 4 + 1], uu = tab[j * 4 + 2], dyj = tab[j * 4 + 3];
        const Cx bv = bvar ? Cx{Bs[sc * kZP + 2 * j], Bs[sc * kZP + 2 * j + 1]} : bc[i];
        const Cx cv = cvar ? Cx{Cs[sc * kZP + 2 * j], Cs[sc * kZP + 2 * j + 1]} : cc[i];
        // g_j = conj(a_{j+1}) g_{j+1} + 2 dy_j conj(C_j)
        gg = cmul(cconj(anx), gg);
        gg.r = fmaf(2.0f * dyj, cv.r, gg.r);
        gg.i = fmaf(-2.0f * dyj, cv.i, gg.i);
        if (!ok) gg = {0.0f, 0.0f};
        const float t1 = gg.r * bv.r + gg.i * bv.i;  // Re(conj(g) B)
        ddl_p[j] = fmaf(uu, t1, ddl_p[j]);
        du_p[j] = fmaf(dl, t1, du_p[j]);
        const Cx xp = j > 0 ? xs[j > 0 ? j - 1 : 0] : x0;
        const Cx ga = cmul(gg, cconj(xp));          // packed gradient of a_j
        const Cx aa = cmul(Cx{arn[i], ai[i]}, as[j]);  // A a_j
        ddl_p[j] += ga.r * aa.r + ga.i * aa.i;        // Re(conj(ga) A a_j)
        const Cx ca = cmul(cconj(as[j]), ga);
        dAa.r = fmaf(dl, ca.r, dAa.r);
        dAa.i = fmaf(dl, ca.i, dAa.i);
        gB[2 * j] = dv * gg.r;
        gB[2 * j + 1] = dv * gg.i;
        gC[2 * j] = 2.0f * dyj * xs[j].r;
        gC[2 * j + 1] = -2.0f * dyj * xs[j].i;
        if (!ok) {
          gC[2 * j] = 0.0f;
          gC[2 * j + 1] = 0.0f;
        }
        anx = as[j];
      }
      gs[i] = gg;
      an[i] = anx;
      accA[i] = dAa;
      if (!bvar) {
#pragma unroll
        for (int j = 0; j < kZT; ++j) {
          dBa.r += gB[2 * j];
          dBa.i += gB[2 * j + 1];
        }
        accB[i] = dBa;
      }
      if (!cvar) {
#pragma unroll
        for (int j = 0; j < kZT; ++j) {
          dCa.r += gC[2 * j];
          dCa.i += gC[2 * j + 1];
        }
        accC[i] = dCa;
      }
      if (bvar || cvar) {
        // the workgroup's channels' rows of this state, added in channel
        // order; channels past the group's end add 0
        if (bvar) {
#pragma unroll
          for (int k = 0; k < 2 * kZT; k += 4)
            *reinterpret_cast<float4*>(&gbB[(wave * 64 + lane) * 32 + k]) =
                ch_ok ? make_float4(gB[k], gB[k + 1], gB[k + 2], gB[k + 3]) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (cvar) {
#pragma unroll
          for (int k = 0; k < 2 * kZT; k += 4)
            *reinterpret_cast<float4*>(&gbC[(wave * 64 + lane) * 32 + k]) =
                ch_ok ? make_float4(gC[k], gC[k + 1], gC[k + 2], gC[k + 3]) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        __syncthreads();
        {
          constexpr int WPT = LPC * 32 / 256;               // words per thread
          const int rs = tid / (32 / WPT), q8 = (tid % (32 / WPT)) * WPT;  // state lane, first word
          const int st = rs + LPC * i;
          if (st < p.dstate) {
            const int64_t row = ((((int64_t)tile * p.batch + b) * p.ngroups + g) * p.dstate + st) * (2 * (int64_t)p.seqlen);
            for (int v = 0; v < 2; ++v) {
              if (v == 0 ? !bvar : !cvar) continue;
              const float* gbuf = v == 0 ? gbB : gbC;
              float* part = v == 0 ? p.dB_part : p.dC_part;
#pragma unroll
              for (int k = 0; k < WPT; ++k) {
                const int w = q8 + k;  // (re, im) word of step w / 2
                float sum = gbuf[rs * 32 + w];
#pragma unroll
                for (int ch = 1; ch < kZW * CPW; ++ch)
                  sum += gbuf[((ch / CPW) * 64 + (ch % CPW) * LPC + rs) * 32 + w];
                if ((w >> 1) < nst) part[row + 2 * (int64_t)l0 + w] = sum;
              }
            }
          }
        }
        __syncthreads();
      }
    }
    // per-step sums over the wave's states
    const float ddl = zlane_sum<LPC>(ddl_p, yb, lane);
    const float dus = zlane_sum<LPC>(du_p, yb, lane);
    if (sl < nst && ch_ok) {
      float dd = ddl;
      if (p.softplus && draw <= 20.0f) dd = ddl * sigmoid_f32(draw);
      static_cast<TU*>(p.du)[orow + l0 + sl] = from_f32<TU>(fmaf(dskip, dy, dus));
      static_cast<TD*>(p.ddelta)[orow + l0 + sl] = from_f32<TD>(dd);
      dbias_acc += dd;
    }
  }
  // per-batch partials
#pragma unroll
  for (int i = 0; i < KS; ++i) {
    const int s = sl + LPC * i;
    if (s < p.dstate && ch_ok) {
      const int64_t e = 2 * (((int64_t)b * p.dim + d) * p.dstate + s);
      p.dA_part[e] = accA[i].r;
      p.dA_part[e + 1] = accA[i].i;
      if (!bvar) {
        p.dBc_part[e] = accB[i].r;
        p.dBc_part[e + 1] = accB[i].i;
      }
      if (!cvar) {
        p.dCc_part[e] = accC[i].r;
        p.dCc_part[e + 1] = accC[i].i;
      }
    }
  }
  // dD / ddelta_bias: lanes 0..15 of a channel hold per-lane sums over their
  // steps; add them in lane order through the transpose buffer
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
  if (sl < kZT) {
    yb[2 * kZT * cw + sl] = dD_acc;
    yb[2 * kZT * cw + kZT + sl] = dbias_acc;
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
  if (sl == 0 && ch_ok) {
    float sD = 0.0f, sb = 0.0f;
    for (int j = 0; j < kZT; ++j) {
      sD += yb[2 * kZT * cw + j];
      sb += yb[2 * kZT * cw + kZT + j];
    }
    p.dD_part[(int64_t)b * p.dim + d] = sD;
    p.dbias_part[(int64_t)b * p.dim + d] = sb;
  }
}

// Fixed-order sums of the backward's partials.
struct ZFin {
  const float *dA_part, *dD_part, *dbias_part, *dBc_part, *dCc_part, *dB_part, *dC_part;
  float *dA, *dD, *dbias, *dBc, *dCc;
  void *dB, *dC;  // input-dependent: [batch, ngroups, dstate, 2 seqlen] in the B / C type
  int batch, dim, dstate, ngroups, tiles, seqlen;
};

__global__ void __launch_bounds__(256) scan_complex_finish_kernel(ZFin f) {
  const int64_t n1 = (int64_t)f.dim * f.dstate;  // complex entries of dA
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n1; e += (int64_t)gridDim.x * 256) {
    float ar = 0.0f, aim = 0.0f, br = 0.0f, bim = 0.0f, cr = 0.0f, cim = 0.0f;
    for (int b = 0; b < f.batch; ++b) {
      const int64_t q = 2 * ((int64_t)b * n1 + e);
      ar += f.dA_part[q];
      aim += f.dA_part[q + 1];
      if (f.dBc) {
        br += f.dBc_part[q];
        bim += f.dBc_part[q + 1];
      }
      if (f.dCc) {
        cr += f.dCc_part[q];
        cim += f.dCc_part[q + 1];
      }
    }
    f.dA[2 * e] = ar;
    f.dA[2 * e + 1] = aim;
    if (f.dBc) {
      f.dBc[2 * e] = br;
      f.dBc[2 * e + 1] = bim;
    }
    if (f.dCc) {
      f.dCc[2 * e] = cr;
      f.dCc[2 * e + 1] = cim;
    }
  }
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < f.dim; e += (int64_t)gridDim.x * 256) {
    float sD = 0.0f, sb = 0.0f;
    for (int b = 0; b < f.batch; ++b) {
      sD += f.dD_part[(int64_t)b * f.dim + e];
      sb += f.dbias_part[(int64_t)b * f.dim + e];
    }
    if (f.dD) f.dD[e] = sD;
    if (f.dbias) f.dbias[e] = sb;
  }
}

template <typename TBC>
__global__ void __launch_bounds__(256) scan_complex_bc_sum_kernel(ZFin f) {
  const int64_t row = 2 * (int64_t)f.seqlen;
  const int64_t n = (int64_t)f.batch * f.ngroups * f.dstate * row;
  const int64_t tstride = n;  // partial rows of one channel tile
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    if (f.dB) {
      float s = 0.0f;
      for (int t = 0; t < f.tiles; ++t) s += f.dB_part[(int64_t)t * tstride + e];
      static_cast<TBC*>(f.dB)[e] = from_f32<TBC>(s);
    }
    if (f.dC) {
      float s = 0.0f;
      for (int t = 0; t < f.tiles; ++t) s += f.dC_part[(int64_t)t * tstride + e];
      static_cast<TBC*>(f.dC)[e] = from_f32<TBC>(s);
    }
  }
}

int zks(int dstate) { return (dstate + 63) / 64; }

template <typename TU, typename TD, typename TBC, int KS, int LPC = 64>
void launch_fwd_ks(const ScanParams& p, size_t bytes, int grid, hipStream_t s) {
  auto kernel = mamba_scan_complex_fwd_kernel<TU, TD, TBC, KS, LPC>;
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  kernel<<<dim3(grid), dim3(256), bytes, s>>>(p);
}

template <typename TU, typename TD, typename TBC, int KS, int LPC = 64>
void launch_bwd_ks(const ScanParams& p, size_t bytes, int grid, hipStream_t s) {
  auto kernel = mamba_scan_complex_bwd_kernel<TU, TD, TBC, KS, LPC>;
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  kernel<<<dim3(grid), dim3(256), bytes, s>>>(p);
}

template <typename TU, typename TD, typename TBC>
void zfwd(const ScanParams& p, hipStream_t s) {
  const ZLayout L = zlayout(p.dstate, !p.b_const, !p.c_const, false);
  const size_t bytes = (size_t)L.total * 4;
  const int grid = p.batch * p.ngroups * p.tiles_per_group;
  if (zlpc(p.dstate) == 16) {
    launch_fwd_ks<TU, TD, TBC, 1, 16>(p, bytes, grid, s);
    return;
  }
  switch (zks(p.dstate)) {
    case 1: launch_fwd_ks<TU, TD, TBC, 1>(p, bytes, grid, s); break;
    case 2: launch_fwd_ks<TU, TD, TBC, 2>(p, bytes, grid, s); break;
    case 3: launch_fwd_ks<TU, TD, TBC, 3>(p, bytes, grid, s); break;
    default: launch_fwd_ks<TU, TD, TBC, 4>(p, bytes, grid, s); break;
  }
}

template <typename TU, typename TD, typename TBC>
void zbwd(const ScanParams& p, hipStream_t s) {
  const ZLayout L = zlayout(p.dstate, !p.b_const, !p.c_const, true);
  const size_t bytes = (size_t)L.total * 4;
  const int grid = p.batch * p.ngroups * p.tiles_per_group;
  if (zlpc(p.dstate) == 16) {
    launch_bwd_ks<TU, TD, TBC, 1, 16>(p, bytes, grid, s);
    return;
  }
  switch (zks(p.dstate)) {
    case 1: launch_bwd_ks<TU, TD, TBC, 1>(p, bytes, grid, s); break;
    case 2: launch_bwd_ks<TU, TD, TBC, 2>(p, bytes, grid, s); break;
    case 3: launch_bwd_ks<TU, TD, TBC, 3>(p, bytes, grid, s); break;
    default: launch_bwd_ks<TU, TD, TBC, 4>(p, bytes, grid, s); break;
  }
}

// (TU, TD, TBC) from the dtype codes: delta and a variable B / C in fp32 or
// u's type (a constant B / C is complex fp32 and takes TBC = float).
template <template <typename, typename, typename> class F>
bool zdispatch(int u_dtype, int delta_dtype, int bc_dtype, const ScanParams& p, hipStream_t s) {
  auto with_u = [&](auto tu) -> bool {
    using TU = decltype(tu);
    const bool d32 = delta_dtype == AK_DTYPE_F32, bc32 = bc_dtype == AK_DTYPE_F32;
    const int uc = std::is_same_v<TU, float> ? AK_DTYPE_F32 : (std::is_same_v<TU, f16> ? AK_DTYPE_F16 : AK_DTYPE_BF16);
    if (!d32 && delta_dtype != uc) return false;
    if (!bc32 && bc_dtype != uc) return false;
    if (d32 && bc32) F<TU, float, float>::run(p, s);
    else if (d32) F<TU, float, TU>::run(p, s);
    else if (bc32) F<TU, TU, float>::run(p, s);
    else F<TU, TU, TU>::run(p, s);
    return true;
  };
  switch (u_dtype) {
    case AK_DTYPE_F32: return with_u(float{});
    case AK_DTYPE_F16: return with_u(f16{});
    default: return with_u(bf16{});
  }
}

template <typename TU, typename TD, typename TBC>
struct ZFwd {
  static void run(const ScanParams& p, hipStream_t s) { zfwd<TU, TD, TBC>(p, s); }
};
template <typename TU, typename TD, typename TBC>
struct ZBwd {
  static void run(const ScanParams& p, hipStream_t s) { zbwd<TU, TD, TBC>(p, s); }
};

size_t zalign(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

ZWs scan_complex_bwd_ws(int64_t batch, int64_t dim, int64_t seqlen, int64_t dstate, int64_t ngroups,
                        int bc_flags) {
  ZWs w{};
  const int64_t cpg = dim / ngroups;
  const int64_t tiles = (cpg + zcpb((int)dstate) - 1) / zcpb((int)dstate);
  const int64_t nck = (seqlen + kCk - 1) / kCk;
  w.ck = zalign((size_t)(batch * nck * dim * dstate) * 8);
  w.prez = zalign((size_t)(batch * dim * seqlen) * 4);
  w.partB = (bc_flags & AK_SCAN_B_CONST) ? 0 : zalign((size_t)(tiles * batch * ngroups * dstate * 2 * seqlen) * 4);
  w.partC = (bc_flags & AK_SCAN_C_CONST) ? 0 : zalign((size_t)(tiles * batch * ngroups * dstate * 2 * seqlen) * 4);
  w.dA = zalign((size_t)(batch * dim * dstate) * 8);
  w.dD = zalign((size_t)(batch * dim) * 4);
  w.dBc = (bc_flags & AK_SCAN_B_CONST) ? w.dA : 0;
  w.dCc = (bc_flags & AK_SCAN_C_CONST) ? w.dA : 0;
  w.total = w.ck + w.prez + w.partB + w.partC + w.dA + 2 * w.dD + w.dBc + w.dCc;
  return w;
}

void launch_scan_complex_zero(int dim, int dstate, float* dA, float* dD, float* ddelta_bias,
                              float* dBc, float* dCc, hipStream_t s) {
  ZFin f{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, dA, dD, ddelta_bias, dBc, dCc,
         nullptr, nullptr, 0, dim, dstate, 1, 0, 0};
  scan_complex_finish_kernel<<<dim3(64), dim3(256), 0, s>>>(f);
}

int launch_scan_complex_fwd(ScanParams p, int u_dtype, int delta_dtype, int bc_dtype, hipStream_t s) {
  p.tiles_per_group = (p.ch_per_group + zcpb(p.dstate) - 1) / zcpb(p.dstate);
  if ((int64_t)p.batch * p.ngroups * p.tiles_per_group > 0x7FFFFFFF) return 1;
  return zdispatch<ZFwd>(u_dtype, delta_dtype, bc_dtype, p, s) ? 0 : 1;
}

int launch_scan_complex_bwd(ScanParams p, const ZWs& ws, void* workspace, bool saved, int u_dtype,
                            int delta_dtype, int bc_dtype, void* dB, void* dC, float* dA, float* dD,
                            float* ddelta_bias, hipStream_t s) {
  p.tiles_per_group = (p.ch_per_group + zcpb(p.dstate) - 1) / zcpb(p.dstate);
  if ((int64_t)p.batch * p.ngroups * p.tiles_per_group > 0x7FFFFFFF) return 1;
  char* w = static_cast<char*>(workspace);
  size_t off = 0;
  auto take = [&](size_t bytes) { float* q = bytes ? reinterpret_cast<float*>(w + off) : nullptr; off += bytes; return q; };
  float* ck = take(ws.ck);
  float* prez = take(ws.prez);
  p.dB_part = take(ws.partB);
  p.dC_part = take(ws.partC);
  p.dA_part = take(ws.dA);
  p.dD_part = take(ws.dD);
  p.dbias_part = take(ws.dD);
  p.dBc_part = take(ws.dBc);
  p.dCc_part = take(ws.dCc);
  if (!saved) {
    // re-run the forward for the 16-step states and the pre-gate output
    ScanParams f = p;
    f.out = nullptr;
    f.last_state = nullptr;
    f.chunk_states = nullptr;
    f.ck = ck;
    f.out_prez = p.z ? prez : nullptr;
    f.o_bs = (int64_t)p.dim * p.seqlen;
    f.o_ds = p.seqlen;
    if (!zdispatch<ZFwd>(u_dtype, delta_dtype, bc_dtype, f, s)) return 1;
    p.ck = ck;
    p.out_prez = f.out_prez;
  }
  if (!zdispatch<ZBwd>(u_dtype, delta_dtype, bc_dtype, p, s)) return 1;
  ZFin f{p.dA_part, p.dD_part, p.dbias_part, p.dBc_part, p.dCc_part, p.dB_part, p.dC_part,
         dA, dD, ddelta_bias, p.b_const ? static_cast<float*>(dB) : nullptr,
         p.c_const ? static_cast<float*>(dC) : nullptr,
         p.b_const ? nullptr : dB, p.c_const ? nullptr : dC,
         p.batch, p.dim, p.dstate, p.ngroups, p.tiles_per_group, p.seqlen};
  scan_complex_finish_kernel<<<dim3(256), dim3(256), 0, s>>>(f);
  if (!p.b_const || !p.c_const) {
    switch (bc_dtype) {
      case AK_DTYPE_F32: scan_complex_bc_sum_kernel<float><<<dim3(1024), dim3(256), 0, s>>>(f); break;
      case AK_DTYPE_F16: scan_complex_bc_sum_kernel<f16><<<dim3(1024), dim3(256), 0, s>>>(f); break;
      default: scan_complex_bc_sum_kernel<bf16><<<dim3(1024), dim3(256), 0, s>>>(f); break;
    }
  }
  return 0;
}

}  // namespace ak
