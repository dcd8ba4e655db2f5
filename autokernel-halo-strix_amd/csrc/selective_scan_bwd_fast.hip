// Reverse pass of the Mamba-1 selective-scan backward for whole-tile shapes
// (sequence length a multiple of 64, channels per group a multiple of 16,
// 4-element aligned rows, every buffer extent below 2 GiB).
//
// The arithmetic and its order are those of the general reverse pass
// (mamba_scan_bwd_kernel in selective_scan.hip, which documents the
// recurrence), so du, ddelta, dz, dA, dD and ddelta_bias have the same bits.
// Where the grid still fills the GPU, a workgroup takes 32 channels (8 waves)
// instead of 16: it then writes one dB / dC partial row per 32 channels, half
// the partial-sum traffic, and the sums over channels are added in another
// order (dB / dC equal to rounding, still deterministic). What else differs
// is the data movement and the control flow:
// * every global access goes through a wave-uniform buffer resource based at
//   the workgroup's first channel, with per-lane 32-bit offsets fixed for the
//   whole pass and the tile offset in the scalar offset: no 64-bit address
//   arithmetic per tile (the general pass issues 48 scalar loads per lane
//   and tile, each with its own address computation);
// * a step's delta', delta' u and dy are formed once, by the lane that also
//   writes the step's du / ddelta, and reach the block's 16 state lanes
//   through a small LDS table read back as float4 broadcasts: the multiplies
//   by them are plain VALU operations rather than DPP row broadcasts, which
//   take about twice the issue time on gfx950; each block's loads are issued
//   one block ahead;
// * the gate and the saved-states dz (kDz: the forward's pre-gate output is
//   given, so dz is formed here) are compile-time choices, and whole tiles
//   need no bounds tests, so each 16-step block is one basic block the
//   scheduler can interleave;
// * du, ddelta and dz are kept for a whole tile and stored as whole row
//   segments (four steps per lane) after its last block.
// At the C5 shape (batch 4, dim 2048, seqlen 4096, dstate 16) the pass takes
// about 435 us with 16-channel workgroups (579 us for the general one on the
// same box) and 1.5% less with 32-channel ones, whose partial sums then read
// 134 MB instead of 268 MB.
#include "scan_buffer.h"

namespace ak {
namespace {

// kWv waves (4 or 8) of 4 channels each per workgroup.
template <typename TU, typename TD, typename TBC, bool kSoftplus, bool kGate, bool kDz, int kWv>
__global__ void __launch_bounds__(64 * kWv)
mamba_scan_bwd_fast_kernel(ScanParams p) {
  static_assert(kWv == 4 || kWv == 8, "16 or 32 channels per workgroup");
  constexpr int kCh = 4 * kWv;  // channels per workgroup
  __shared__ float Bs[16 * kBStride];
  __shared__ float Cs[16 * kBStride];
  __shared__ __align__(16) float tbuf[kWv][4 * kTC];     // per wave: (g B, A w)[c][j][n]
  __shared__ float wbuf[kWv][64 * kWP];                  // per wave: (dB, dC) channel sums [lane][pair]

  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int c = lane / 16;
  const int n = lane % 16;
  const int tpg = p.tiles_per_group;  // whole kCh-channel tiles
  const int per_batch = p.ngroups * tpg;
  const int b = blockIdx.x / per_batch;
  const int g = (blockIdx.x % per_batch) / tpg;
  const int tile = blockIdx.x % tpg;
  const int d0 = g * p.ch_per_group + tile * kCh;
  const int wc = wave * 4 + c;
  const int d = d0 + wc;
  const bool n_ok = n < p.dstate;

  const float a_nat = n_ok ? p.A[(int64_t)d * p.A_ds + n] : 0.0f;
  const float a_scaled = a_nat * kLog2e;
  const float dbias = p.delta_bias ? p.delta_bias[d] : 0.0f;
  const float dskip = p.D ? p.D[d] : 0.0f;

  const uint32_t L = (uint32_t)p.seqlen;
  auto row_rsrc = [&](const void* base, int64_t bs, int64_t ds, int esz) {
    const char* q = static_cast<const char*>(base) + ((int64_t)b * bs + (int64_t)d0 * ds) * esz;
    return make_rsrc(q, (uint32_t)(((kCh - 1) * ds + L) * esz));
  };
  const Rsrc rs_u = row_rsrc(p.u, p.u_bs, p.u_ds, sizeof(TU));
  const Rsrc rs_d = row_rsrc(p.delta, p.d_bs, p.d_ds, sizeof(TD));
  const Rsrc rs_go = row_rsrc(p.dout, p.go_bs, p.go_ds, sizeof(TU));
  const Rsrc rs_z = kGate ? row_rsrc(p.z, p.z_bs, p.z_ds, sizeof(TU)) : rs_u;
  const Rsrc rs_y = kDz ? row_rsrc(p.out_prez, p.o_bs, p.o_ds, sizeof(TU)) : rs_u;
  const Rsrc rs_du = row_rsrc(p.du, p.o_bs, p.o_ds, sizeof(TU));
  const Rsrc rs_dd = row_rsrc(p.ddelta, p.o_bs, p.o_ds, sizeof(TD));
  const Rsrc rs_dz = (kGate && kDz) ? row_rsrc(p.dz, p.o_bs, p.o_ds, sizeof(TU)) : rs_du;
  const uint32_t bc_bytes_B = (uint32_t)(((p.dstate - 1) * p.B_ns + L) * sizeof(TBC));
  const uint32_t bc_bytes_C = (uint32_t)(((p.dstate - 1) * p.C_ns + L) * sizeof(TBC));
  const Rsrc rs_B = make_rsrc(static_cast<const TBC*>(p.B) + (int64_t)b * p.B_bs + (int64_t)g * p.B_gs, bc_bytes_B);
  const Rsrc rs_C = make_rsrc(static_cast<const TBC*>(p.C) + (int64_t)b * p.C_bs + (int64_t)g * p.C_gs, bc_bytes_C);
  // saved states [batch, nchunks, dim, dstate]: the workgroup's kCh x dstate block of a chunk
  const int64_t ck_cs = (int64_t)p.dim * p.dstate;  // floats per chunk
  const Rsrc rs_ck = make_rsrc(p.ck + (int64_t)b * p.nchunks * ck_cs + (int64_t)d0 * p.dstate,
                               (uint32_t)(((int64_t)(p.nchunks - 1) * ck_cs + kCh * p.dstate) * 4));

  const uint32_t vo_d1 = (uint32_t)(wc * p.d_ds + n) * sizeof(TD);
  const uint32_t vo_u1 = (uint32_t)(wc * p.u_ds + n) * sizeof(TU);
  const uint32_t vo_g1 = (uint32_t)(wc * p.go_ds + n) * sizeof(TU);
  const uint32_t vo_z1 = kGate ? (uint32_t)(wc * p.z_ds + n) * sizeof(TU) : vo_u1;
  const uint32_t vo_o1 = (uint32_t)(wc * p.o_ds + n) * sizeof(TU);   // y (out_prez)
  // B / C staging by waves 0-3: state sn, steps 4 q .. 4 q + 3
  const bool stager = wave < 4;
  const int sn = (tid / 16) % 16, q = tid % 16;
  const int sn_c = min(sn, p.dstate - 1);
  const uint32_t vo_B = (uint32_t)(sn_c * p.B_ns + 4 * q) * sizeof(TBC);
  const uint32_t vo_C = (uint32_t)(sn_c * p.C_ns + 4 * q) * sizeof(TBC);
  const uint32_t vo_ck = (uint32_t)(wc * p.dstate + min(n, p.dstate - 1)) * 4u;

  float* tb = tbuf[wave];
  float* wb = wbuf[wave];
  // Per-wave tbuf use, channel c at c * kTC: the (g B, A w)[j][n] transpose
  // in floats 0..31 of each 36-float step row; the block's per-step table
  // (delta', delta' u, dy of its 16 steps, float4 slot s = 4 q + i: quantity
  // q, steps 4 i .. 4 i + 3) in the row pads, floats 32..35 of row s (row
  // s + 1 for channels 2, 3, so the four channels' slots fall on disjoint
  // banks).
  const int tab = c * kTC + (c >= 2 ? kTJ : 0) + 32;

  // one block's per-step values (step 16 blk + n of channel wc) and the
  // state before the block
  struct Blk {
    Raw1<TD> dr;
    Raw1<TU> ur, gr, zr, yr;
    uint32_t ck;
  };
  auto load_blk = [&](int t, int blk, Blk& r) {
    // wave-uniform, and pinned to an SGPR: for block 0 the compiler shares
    // max(t - 1, 0) with the divergent B / C staging branch, and as a VGPR
    // value the scalar offsets below became one waterfall loop per load
    // (about 1.7% of the pass at the C5 shape)
    const uint32_t l = (uint32_t)__builtin_amdgcn_readfirstlane(t * kScanT + 16 * blk);
    r.dr = bload1<TD>(rs_d, vo_d1, l * sizeof(TD));
    r.ur = bload1<TU>(rs_u, vo_u1, l * sizeof(TU));
    r.gr = bload1<TU>(rs_go, vo_g1, l * sizeof(TU));
    if constexpr (kGate) r.zr = bload1<TU>(rs_z, vo_z1, l * sizeof(TU));
    if constexpr (kGate && kDz) r.yr = bload1<TU>(rs_y, vo_o1, l * sizeof(TU));
    r.ck = __builtin_amdgcn_raw_buffer_load_b32(rs_ck, (int)vo_ck, (int)((l / kCk) * (uint32_t)ck_cs * 4u), 0);
  };

  float gs = 0.0f, a_next = 0.0f, dA_acc = 0.0f, dD_acc = 0.0f, dbias_acc = 0.0f;
  const int nt = p.seqlen / kScanT;
  Raw4<TBC> bv{}, cv{};
  if (stager) {
    bv = bload4<TBC>(rs_B, vo_B, (uint32_t)(nt - 1) * kScanT * sizeof(TBC));
    cv = bload4<TBC>(rs_C, vo_C, (uint32_t)(nt - 1) * kScanT * sizeof(TBC));
  }
  Blk pb;
  load_blk(nt - 1, 3, pb);
  // A tile's du / ddelta / dz, one value per 16-step block (step 16 blk + n
  // of channel wc), stored once the tile is done as whole row segments: four
  // consecutive steps per lane, so each channel row of the tile is one
  // 128-byte (2-byte types) or 256-byte (fp32) store. Stored per block, each
  // row went out as 32- or 64-byte segments a block apart, and the partially
  // written lines left L2 between them: at the C5 shape that cost about 47 MB
  // of extra fetch and 61 MB of extra writes per pass.
  float st_du[4], st_dd[4], st_dz[4];
  const uint32_t vo_o4 = (uint32_t)(wc * p.o_ds + 4 * n) * sizeof(TU);
  const uint32_t vo_dd4 = (uint32_t)(wc * p.o_ds + 4 * n) * sizeof(TD);
  for (int t = nt - 1; t >= 0; --t) {
    const int l0 = t * kScanT;
    __syncthreads();
    if (stager) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const bool ok = sn < p.dstate;
        Bs[sn * kBStride + 4 * q + k] = ok ? raw4_f32<TBC>(bv, k) : 0.0f;
        Cs[sn * kBStride + 4 * q + k] = ok ? raw4_f32<TBC>(cv, k) : 0.0f;
      }
      const uint32_t ln = (uint32_t)max(t - 1, 0) * kScanT;
      bv = bload4<TBC>(rs_B, vo_B, ln * sizeof(TBC));
      cv = bload4<TBC>(rs_C, vo_C, ln * sizeof(TBC));
    }
    asm volatile("" ::: "memory");
    __syncthreads();

    auto block = [&](auto blk_c) {
      constexpr int BLK = decltype(blk_c)::value;
      const Blk cb = pb;
      // the next block's values: one block (about 2 us) of latency cover
      if constexpr (BLK > 0) load_blk(t, BLK - 1, pb);
      else load_blk(max(t - 1, 0), 3, pb);
      asm volatile("" ::: "memory");
      // step 16 BLK + n: delta', dy = dout silu(z) (dout without a gate)
      const float go = raw_f32<TU>(cb.gr);
      float dyv = go, zv = 0.0f, sg = 0.0f;
      if constexpr (kGate) {
        zv = raw_f32<TU>(cb.zr);
        sg = sigmoid_f32(zv);
        dyv = go * zv * sg;
      }
      const float uv = raw_f32<TU>(cb.ur);
      const float x = raw_f32<TD>(cb.dr) + dbias;
      const float dlt = kSoftplus ? softplus_f32(x) : x;
      tb[tab + (n >> 2) * kTJ + (n & 3)] = dlt;
      tb[tab + (4 + (n >> 2)) * kTJ + (n & 3)] = dlt * uv;
      tb[tab + (8 + (n >> 2)) * kTJ + (n & 3)] = dyv;
      __builtin_amdgcn_wave_barrier();
      auto tab4 = [&](int slot) { return *reinterpret_cast<const float4*>(&tb[tab + slot * kTJ]); };
      auto el = [](const float4& v, int k) { return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w; };

      const float hstart = n_ok ? __builtin_bit_cast(float, cb.ck) : 0.0f;
      float bt[16], ct[16], as[16], hs[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        bt[j] = Bs[n * kBStride + 16 * BLK + j];
        ct[j] = Cs[n * kBStride + 16 * BLK + j];
      }
      float xv[16];
      // delta' and delta' u of the block's steps, kept for the reverse sweep
      // (re-reading them there costs more LDS time than the 32 VGPRs)
      float4 fvd[4], fvu[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 vd = tab4(i), vu = tab4(4 + i);
        fvd[i] = vd;
        fvu[i] = vu;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          as[4 * i + k] = el(vd, k) * a_scaled;
          xv[4 * i + k] = el(vu, k) * bt[4 * i + k];
        }
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) as[j] = __builtin_amdgcn_exp2f(as[j]);
      float h = hstart;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        h = fmaf(as[j], h, xv[j]);
        hs[j] = h;
      }
      float pB = 0.0f, pC = 0.0f;
      asm volatile("" ::: "memory");  // the reverse sweep reads the dy table here, not earlier
      float4 gd, gu, gy;
      static_for<0, 16>([&](auto i_c) {
        constexpr int J = 15 - decltype(i_c)::value;
        if constexpr (J % 4 == 3) {
          gd = fvd[J / 4];
          gu = fvu[J / 4];
          gy = tab4(8 + J / 4);
        }
        const float sdj = el(gd, J % 4), suj = el(gu, J % 4), syj = el(gy, J % 4);
        gs = fmaf(gs, a_next, syj * ct[J]);
        a_next = as[J];
        const float hp = J > 0 ? hs[J > 0 ? J - 1 : 0] : hstart;
        const float w = gs * (as[J] * hp);
        // dA += delta' w as an opaque FMA: as plain code the scheduler sinks the
        // whole tile's chain to its end and keeps every w live (274 VGPRs)
        asm("v_fmac_f32 %0, %1, %2" : "+v"(dA_acc) : "v"(sdj), "v"(w));
        const float cB = suj * gs;
        const float cC = syj * hs[J];
        *reinterpret_cast<float2*>(&tb[c * kTC + J * kTJ + 2 * n]) = make_float2(gs * bt[J], a_nat * w);
        if constexpr (J % 2 == 1) {
          pB = cB;
          pC = cC;
        } else {
          const float s_even = swap32_sum(cB, cC);
          const float s_odd = swap32_sum(pB, pC);
          wb[lane * kWP + 8 * BLK + J / 2] = swap16_sum(s_even, s_odd);
        }
      });
      __builtin_amdgcn_wave_barrier();
      asm volatile("" ::: "memory");
      // lane (c, j = n): sum(g B) and sum(A w) over the states of step 16 BLK + n
      float sgb = 0.0f, saw = 0.0f;
#pragma unroll
      for (int s4 = 0; s4 < 8; ++s4) {
        const float4 v = *reinterpret_cast<const float4*>(&tb[c * kTC + n * kTJ + 4 * s4]);
        sgb += v.x + v.z;
        saw += v.y + v.w;
      }
      __builtin_amdgcn_wave_barrier();
      if constexpr (kGate && kDz) st_dz[BLK] = go * raw_f32<TU>(cb.yr) * sg * fmaf(zv, 1.0f - sg, 1.0f);
      float ddl = fmaf(uv, sgb, saw);
      if constexpr (kSoftplus) {
        if (x <= 20.0f) ddl *= sigmoid_f32(x);
      }
      st_du[BLK] = fmaf(dskip, dyv, dlt * sgb);
      st_dd[BLK] = ddl;
      dD_acc = fmaf(dyv, uv, dD_acc);
      dbias_acc += ddl;
    };
    block(std::integral_constant<int, 3>{});
    block(std::integral_constant<int, 2>{});
    block(std::integral_constant<int, 1>{});
    block(std::integral_constant<int, 0>{});
    {
      // the tile's outputs through the wave's transpose buffer (free between
      // tiles): [stream][channel c, pitch 80 floats][step], conflict-free for
      // the b32 writes and the b128 reads
      constexpr int kSP = 80, kSS = 4 * kSP;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        tb[c * kSP + 16 * blk + n] = st_du[blk];
        tb[kSS + c * kSP + 16 * blk + n] = st_dd[blk];
        if constexpr (kGate && kDz) tb[2 * kSS + c * kSP + 16 * blk + n] = st_dz[blk];
      }
      __builtin_amdgcn_wave_barrier();
      asm volatile("" ::: "memory");
      bstore4_at<TU>(rs_du, vo_o4, (uint32_t)l0 * sizeof(TU), *reinterpret_cast<const float4*>(&tb[c * kSP + 4 * n]));
      bstore4_at<TD>(rs_dd, vo_dd4, (uint32_t)l0 * sizeof(TD),
                     *reinterpret_cast<const float4*>(&tb[kSS + c * kSP + 4 * n]));
      if constexpr (kGate && kDz)
        bstore4_at<TU>(rs_dz, vo_o4, (uint32_t)l0 * sizeof(TU),
                       *reinterpret_cast<const float4*>(&tb[2 * kSS + c * kSP + 4 * n]));
      __builtin_amdgcn_wave_barrier();
      asm volatile("" ::: "memory");
    }

    __syncthreads();
    {
      // step l0 + tt, states kPer ng .. kPer ng + kPer - 1: the waves' channel
      // sums added in wave order
      constexpr int kPer = 16 / kWv;
      const int tt = tid % 64, ng = tid / 64;
      const int l = l0 + tt;
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        float* part = v ? p.dC_part : p.dB_part;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
          const int n2 = kPer * ng + i;
          const int Lr = 16 * (2 * v + (tt & 1)) + n2;
          float sum = wbuf[0][Lr * kWP + tt / 2];
#pragma unroll
          for (int w = 1; w < kWv; ++w) sum += wbuf[w][Lr * kWP + tt / 2];
          if (n2 < p.dstate)
            part[((((int64_t)tile * p.batch + b) * p.ngroups + g) * p.dstate + n2) * p.seqlen + l] = sum;
        }
      }
    }
  }
  if (n_ok) p.dA_part[((int64_t)b * p.dim + d) * p.dstate + n] = dA_acc;
  dD_acc = row16_sum(dD_acc);
  dbias_acc = row16_sum(dbias_acc);
  if (n == 0) {
    p.dD_part[(int64_t)b * p.dim + d] = dD_acc;
    p.dbias_part[(int64_t)b * p.dim + d] = dbias_acc;
  }
}

template <typename TU, typename TD, typename TBC>
bool scan_bwd_fast_ok(const ScanParams& p, int wgc) {
  auto al4 = [](const void* ptr, int64_t s0, int64_t s1, size_t esz) {
    return (reinterpret_cast<uintptr_t>(ptr) % (4 * esz)) == 0 && s0 % 4 == 0 && s1 % 4 == 0;
  };
  auto fits = [&](int64_t rows, int64_t pitch, size_t esz) {
    return pitch >= 0 && ((rows - 1) * pitch + p.seqlen) * (int64_t)esz < ((int64_t)1 << 31);
  };
  if (p.seqlen % kScanT != 0 || p.ch_per_group % wgc != 0 || p.dstate > 16) return false;
  if (p.b_const || p.c_const) return false;
  if (!al4(p.u, p.u_bs, p.u_ds, sizeof(TU)) || !al4(p.delta, p.d_bs, p.d_ds, sizeof(TD)) ||
      !al4(p.dout, p.go_bs, p.go_ds, sizeof(TU)))
    return false;
  if (p.z && !al4(p.z, p.z_bs, p.z_ds, sizeof(TU))) return false;
  if (reinterpret_cast<uintptr_t>(p.B) % (4 * sizeof(TBC)) || reinterpret_cast<uintptr_t>(p.C) % (4 * sizeof(TBC)) ||
      p.B_bs % 4 || p.B_gs % 4 || p.B_ns % 4 || p.C_bs % 4 || p.C_gs % 4 || p.C_ns % 4)
    return false;
  if (p.u_bs < 0 || p.d_bs < 0 || p.go_bs < 0 || p.z_bs < 0 || p.o_bs < 0 || p.B_bs < 0 ||
      p.C_bs < 0 || p.B_gs < 0 || p.C_gs < 0)
    return false;
  const int64_t ck_bytes = ((int64_t)(p.nchunks - 1) * p.dim * p.dstate + wgc * p.dstate) * 4;
  if (ck_bytes >= ((int64_t)1 << 31)) return false;
  return fits(wgc, p.u_ds, sizeof(TU)) && fits(wgc, p.d_ds, sizeof(TD)) &&
         fits(wgc, p.go_ds, sizeof(TU)) && fits(wgc, p.o_ds, sizeof(TD)) &&
         (!p.z || fits(wgc, p.z_ds, sizeof(TU))) && fits(p.dstate, p.B_ns, sizeof(TBC)) &&
         fits(p.dstate, p.C_ns, sizeof(TBC));
}

template <typename TU, typename TD, typename TBC>
bool launch_fast(ScanParams& p, hipStream_t s) {
  // 32-channel workgroups when there are at least kWideMinGroups of them
  // (one per CU on MI355X). The threshold is a constant, not the live CU
  // count: the choice fixes the order in which dB / dC are summed over
  // channels, so it depends on the shape alone and the bits of every
  // gradient are the same on any device or partition.
  constexpr int64_t kWideMinGroups = 256;
  const bool wide = p.ch_per_group % 32 == 0 && scan_bwd_fast_ok<TU, TD, TBC>(p, 32) &&
                    (int64_t)p.batch * p.ngroups * (p.ch_per_group / 32) >= kWideMinGroups;
  if (!wide && !scan_bwd_fast_ok<TU, TD, TBC>(p, kScanCh)) return false;
  if (wide) p.tiles_per_group = p.ch_per_group / 32;
  const int grid = p.batch * p.ngroups * p.tiles_per_group;
  const bool gate = p.z != nullptr, dz = gate && p.out_prez != nullptr;
  auto go = [&](auto sp, auto gt, auto dzt) {
    constexpr bool kSp = decltype(sp)::value, kGt = decltype(gt)::value, kDzt = decltype(dzt)::value;
    if (wide)
      mamba_scan_bwd_fast_kernel<TU, TD, TBC, kSp, kGt, kDzt, 8><<<dim3(grid), dim3(512), 0, s>>>(p);
    else
      mamba_scan_bwd_fast_kernel<TU, TD, TBC, kSp, kGt, kDzt, 4><<<dim3(grid), dim3(256), 0, s>>>(p);
  };
  using T = std::true_type;
  using F = std::false_type;
  if (p.softplus) {
    if (dz) go(T{}, T{}, T{});
    else if (gate) go(T{}, T{}, F{});
    else go(T{}, F{}, F{});
  } else {
    if (dz) go(F{}, T{}, T{});
    else if (gate) go(F{}, T{}, F{});
    else go(F{}, F{}, F{});
  }
  return true;
}

template <typename TU>
bool dispatch_fast(ScanParams& p, int u_dtype, int delta_dtype, int bc_dtype, hipStream_t s) {
  const bool d32 = delta_dtype == AK_DTYPE_F32, bc32 = bc_dtype == AK_DTYPE_F32;
  if (!d32 && delta_dtype != u_dtype) return false;
  if (!bc32 && bc_dtype != u_dtype) return false;
  if (d32 && bc32) return launch_fast<TU, float, float>(p, s);
  if (d32) return launch_fast<TU, float, TU>(p, s);
  if (bc32) return launch_fast<TU, TU, float>(p, s);
  return launch_fast<TU, TU, TU>(p, s);
}

}  // namespace

bool launch_scan_bwd_fast(ScanParams& p, int u_dtype, int delta_dtype, int bc_dtype,
                          hipStream_t s) {
  switch (u_dtype) {
    case AK_DTYPE_F32: return dispatch_fast<float>(p, u_dtype, delta_dtype, bc_dtype, s);
    case AK_DTYPE_F16: return dispatch_fast<f16>(p, u_dtype, delta_dtype, bc_dtype, s);
    case AK_DTYPE_BF16: return dispatch_fast<bf16>(p, u_dtype, delta_dtype, bc_dtype, s);
    default: return false;
  }
}

}  // namespace ak
