// Mamba-1 selective scan forward and backward, and the diagonal linear
// recurrence with its backward, gfx950.
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
// folds h[n] * C[n] with 16 FMAs, one block later than the recurrence so
// that the transpose's LDS latency is hidden. B and C are staged per 64-step
// tile in LDS as fp32, converted once per workgroup; each lane reads its
// state's 64 B values once per tile. exp uses exp2 with A pre-scaled by
// log2(e), like the reference kernel (selective_scan_fwd_kernel.cuh:173-177).
// On request the forward also writes y + D u before the gate and, per
// 2048-step chunk, the running prefix (decay product, state) of every state
// (the reference binding's chunk-state tensor x). The backward's design is
// described above mamba_scan_bwd_kernel.
#include "scan_buffer.h"

namespace ak {
namespace {

// kPrep: the preparation pass of the backward. Instead of the output it
// writes the state before every 64-step tile to p.ck and, with a gate,
// dz = dout * y * silu'(z) (y the output before the gate).
template <typename TU, typename TD, typename TBC, bool kPrep = false>
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
  const int64_t go_row = (int64_t)b * p.go_bs + (int64_t)d * p.go_ds;
  const int64_t B_base = (int64_t)b * p.B_bs + (int64_t)g * p.B_gs;
  const int64_t C_base = (int64_t)b * p.C_bs + (int64_t)g * p.C_gs;

  float h = 0.0f;
  float* hb = hbuf[wave];

  // Global loads for one 64-step tile, issued one tile ahead of their use so
  // that their latency hides behind the previous tile's recurrence. They
  // load from clamped, always-valid addresses without conditions and keep
  // the storage type: masking and conversion to fp32 happen at the use, a
  // tile later (a conditional or converting load would have to wait for its
  // data right away).
  struct TileRegs {
    TBC bv[4], cv[4];  // B / C staging: state sn, steps 4q..4q+3
    TD dv[4];          // this lane's broadcast steps 4n..4n+3
    TU uv[4];
    TU uo[4], zo[4];   // output steps 16*blk + n, blk = 0..3
    TU go[4];          // kPrep: dout at the same steps
  };
  const int sn = tid / 16, q = tid % 16;
  const int sn_c = min(sn, p.dstate - 1);
  const int last_l = p.seqlen - 1;
  // without z the gate loads read u instead (unused)
  const TU* const zsrc = static_cast<const TU*>(p.z ? p.z : p.u);
  const int64_t zrow = p.z ? z_row : u_row;
  auto load_tile = [&](int l0, TileRegs& r) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int l = min(l0 + 4 * q + k, last_l);
      r.bv[k] = static_cast<const TBC*>(p.B)[B_base + (int64_t)sn_c * p.B_ns + l];
      r.cv[k] = static_cast<const TBC*>(p.C)[C_base + (int64_t)sn_c * p.C_ns + l];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int l = min(l0 + 4 * n + k, last_l);
      r.dv[k] = static_cast<const TD*>(p.delta)[d_row + l];
      r.uv[k] = static_cast<const TU*>(p.u)[u_row + l];
    }
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int l = min(l0 + 16 * blk + n, last_l);
      r.uo[blk] = static_cast<const TU*>(p.u)[u_row + l];
      r.zo[blk] = zsrc[zrow + l];
      if constexpr (kPrep) r.go[blk] = static_cast<const TU*>(p.dout)[go_row + l];
    }
  };

  // The output reduction of a 16-step block runs one block late: its
  // transpose reads are issued right after the states are written and are
  // consumed after the next block's recurrence, which hides their latency.
  float ph[16] = {}, pc[16] = {};  // pending block: h[c][j][0..15] and C[j][0..15]
  float p_uo = 0.0f, p_zo = 0.0f, p_go = 0.0f;
  int p_l = -1;              // pending output step (-1: none)
  auto finish_pending = [&]() {
    float y = 0.0f;
#pragma unroll
    for (int s = 0; s < 16; ++s) y = fmaf(ph[s], pc[s], y);
    if (ch_ok && p_l >= 0 && p_l < p.seqlen) {
      float o = fmaf(dskip, p_uo, y);
      if constexpr (kPrep) {
        if (p.z) {
          // d(y * silu(z)) / dz = y * s * (1 + z (1 - s)),  s = sigmoid(z)
          const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-p_zo * kLog2e));
          const float dzv = p_go * o * sg * fmaf(p_zo, 1.0f - sg, 1.0f);
          static_cast<TU*>(p.dz)[o_row + p_l] = from_f32<TU>(dzv);
        }
      } else {
        if (p.out_prez) static_cast<TU*>(p.out_prez)[o_row + p_l] = from_f32<TU>(o);
        if (p.z) o *= silu_fast(p_zo);
        static_cast<TU*>(p.out)[o_row + p_l] = from_f32<TU>(o);
      }
    }
  };

  float dsum = 0.0f;  // sum of delta' since step 0 (chunk states)
  TileRegs cur, nxt{};
  load_tile(0, cur);
  for (int l0 = 0; l0 < p.seqlen; l0 += kScanT) {
    __syncthreads();  // previous tile's readers of Bs / Cs are done
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const bool ok = sn < p.dstate && l0 + 4 * q + k < p.seqlen;
      Bs[sn * kBStride + 4 * q + k] = ok ? to_f32(cur.bv[k]) : 0.0f;
      Cs[(4 * q + k) * kCStride + sn] = ok ? to_f32(cur.cv[k]) : 0.0f;
    }
    float dl[4], du[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const bool ok = ch_ok && l0 + 4 * n + k < p.seqlen;
      float dv = to_f32(cur.dv[k]) + dbias;
      if (p.softplus) dv = softplus_f32(dv);
      dl[k] = ok ? dv : 0.0f;
      du[k] = dl[k] * to_f32(cur.uv[k]);
    }
    // wait states between the last VALU write of dl / du and their DPP reads
    asm volatile("s_nop 1"
                 : "+v"(dl[0]), "+v"(dl[1]), "+v"(dl[2]), "+v"(dl[3]), "+v"(du[0]), "+v"(du[1]),
                   "+v"(du[2]), "+v"(du[3]));
    if (l0 + kScanT < p.seqlen) load_tile(l0 + kScanT, nxt);
    // keep the compiler from sinking the prefetch towards its use
    asm volatile("" ::: "memory");
    __syncthreads();
    // B[n][l0 .. l0 + 63] of this lane's state, read once per tile
    float bt[kScanT];
#pragma unroll
    for (int l = 0; l < kScanT; ++l) bt[l] = Bs[n * kBStride + l];

#pragma unroll
    for (int blk = 0; blk < kScanT / 16; ++blk) {
      if (kPrep || p.ck) {
        // state before the block: the reverse pass restarts from it (the
        // forward writes it too when given a checkpoint buffer)
        const int lb = l0 + 16 * blk;
        if (ch_ok && n_ok && lb < p.seqlen)
          p.ck[(((int64_t)b * p.nchunks + lb / kCk) * p.dim + d) * p.dstate + n] = h;
      }
      float hv[16];
      // Steps 16 blk + 4 j4 + k come from lane src = 4 blk + j4 of the row.
      // All decay factors and inputs of the block are formed first (they do
      // not depend on h), then the 16-step FMA chain runs; this keeps the
      // exp results away from their uses (no hazard wait states).
      float av[16], xv[16];
      auto steps4 = [&](auto src_c, int j4) {
        constexpr int kSrc = decltype(src_c)::value;
#pragma unroll
        for (int k = 0; k < 4; ++k) av[4 * j4 + k] = mul_bcast<kSrc>(dl[k], a_scaled);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          xv[4 * j4 + k] = mul_bcast<kSrc>(du[k], bt[16 * blk + 4 * j4 + k]);
      };
      switch (blk) {
        case 0:
          steps4(std::integral_constant<int, 0>{}, 0); steps4(std::integral_constant<int, 1>{}, 1);
          steps4(std::integral_constant<int, 2>{}, 2); steps4(std::integral_constant<int, 3>{}, 3);
          break;
        case 1:
          steps4(std::integral_constant<int, 4>{}, 0); steps4(std::integral_constant<int, 5>{}, 1);
          steps4(std::integral_constant<int, 6>{}, 2); steps4(std::integral_constant<int, 7>{}, 3);
          break;
        case 2:
          steps4(std::integral_constant<int, 8>{}, 0); steps4(std::integral_constant<int, 9>{}, 1);
          steps4(std::integral_constant<int, 10>{}, 2); steps4(std::integral_constant<int, 11>{}, 3);
          break;
        default:
          steps4(std::integral_constant<int, 12>{}, 0); steps4(std::integral_constant<int, 13>{}, 1);
          steps4(std::integral_constant<int, 14>{}, 2); steps4(std::integral_constant<int, 15>{}, 3);
          break;
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) av[j] = __builtin_amdgcn_exp2f(av[j]);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        h = fmaf(av[j], h, xv[j]);
        hv[j] = h;
      }
      // Order: this block's recurrence, then the previous block's output
      // (whose transpose reads are by now complete), then this block's
      // transpose. The empty asm statement (h must be final before it) and
      // the scheduling barrier pin that order.
      asm volatile("" : "+v"(h));
      __builtin_amdgcn_sched_barrier(0);
      finish_pending();  // previous block's output
      // Transpose through LDS: hbuf[c][j][n] = h at step j of this block.
#pragma unroll
      for (int j = 0; j < 16; ++j) hb[c * kHC + j * kHJ + n] = hv[j];
      __builtin_amdgcn_wave_barrier();
      // Lane (c, j=n) owns step j of channel c: its 16 states and C values.
#pragma unroll
      for (int s2 = 0; s2 < 16; ++s2) {
        ph[s2] = hb[c * kHC + n * kHJ + s2];
        pc[s2] = Cs[(16 * blk + n) * kCStride + s2];
      }
      __builtin_amdgcn_wave_barrier();
      p_uo = to_f32(cur.uo[blk]);
      p_zo = p.z ? to_f32(cur.zo[blk]) : 0.0f;
      if constexpr (kPrep) p_go = to_f32(cur.go[blk]);
      p_l = l0 + 16 * blk + n;
    }
    if (!kPrep && p.chunk_states) {
      // the channel's delta' over the tile (invalid steps hold 0)
      dsum += row16_sum((dl[0] + dl[1]) + (dl[2] + dl[3]));
      const int l1 = l0 + kScanT;
      if ((l1 % kXChunk == 0 || l1 >= p.seqlen) && ch_ok && n_ok) {
        float* xs = p.chunk_states +
                    ((((int64_t)b * p.dim + d) * p.xchunks + (l1 - 1) / kXChunk) * p.dstate + n) * 2;
        xs[0] = __builtin_amdgcn_exp2f(a_scaled * dsum);
        xs[1] = h;
      }
    }
    cur = nxt;
  }
  finish_pending();
  if (!kPrep && p.last_state && ch_ok && n_ok) {
    p.last_state[((int64_t)b * p.dim + d) * p.dstate + n] = h;
  }
}

// ---------------------------------------------------------------------------
// Fast path: seqlen a multiple of 64, channels per group a multiple of 16,
// 4-element (8- or 16-byte) aligned rows, every per-workgroup extent below
// 2 GiB (checked on the host). Same lane decomposition and arithmetic as
// mamba_scan_fwd_kernel, with
// * buffer loads and stores through wave-uniform resources whose base is the
//   workgroup's first channel: per-lane 32-bit offsets are fixed for the
//   whole scan and the tile offset rides in the scalar offset, so no address
//   arithmetic runs per tile; delta and u come in one 8/16-byte load per
//   lane and tile, B and C in one each per thread;
// * B / C staging double-buffered in LDS with one workgroup barrier per
//   tile: tile t + 1 is written while tile t is read, from registers loaded
//   a tile earlier;
// * the output dot product split into four independent FMA chains;
// * softplus chosen at compile time (as a run-time branch the compiler
//   if-converts it and evaluates log1p(exp(x)) on every tile).
// ---------------------------------------------------------------------------
// kPrep: the backward's preparation pass (as in mamba_scan_fwd_kernel). The
// forward's optional outputs (gate, pre-gate output, checkpoints, chunk
// states) are tested at run time. For dstate <= 16 the forwards run on
// mamba_scan_split_kernel (below), which also has variants with those outputs
// fixed at compile time (the run-time tests split the tile loop into basic
// blocks that the scheduler cannot interleave across: about 8% of the kernel
// at the C5 shape); this kernel is launched for dstate 17-64 (kRPC > 1) and as
// the preparation pass without a gate.
//
// The forward variants of mamba_scan_split_kernel: kFwdAny tests the outputs'
// pointers at run time; kFwdLean has a gate z and none of out_prez,
// checkpoints or chunk states (inference); kFwdTrain has a gate, out_prez and
// checkpoints but no chunk states (the training forward that keeps its
// states).
enum { kFwdAny = 0, kFwdLean = 1, kFwdTrain = 2 };

// kRPC (forward only): 16-lane rows per channel, for dstate up to 16 * kRPC.
// With kRPC > 1 a channel's states span kRPC rows of its wave (state = 16 *
// row-in-channel + lane); each row sums its 16 states' outputs through the LDS
// transpose as with one row, and the rows' partials are added with permlane
// swaps. A workgroup then holds 16 / kRPC channels, and the larger B / C
// staging is single-buffered (two barriers per tile) so that two workgroups
// still fit in a CU's LDS.
template <typename TU, typename TD, typename TBC, bool kSoftplus, bool kPrep = false, int kRPC = 1>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu((kRPC == 4 && sizeof(TBC) == 2) || kRPC == 2 ? 3 : 1)))
mamba_scan_fast_kernel(ScanParams p) {
  static_assert(kRPC == 1 || kRPC == 2 || kRPC == 4, "1, 2 or 4 rows per channel");
  static_assert(!(kPrep && kRPC != 1), "the preparation pass has 16 states");
  constexpr int kNS = 16 * kRPC;                         // state slots per channel
  constexpr int kCPW = 4 / kRPC;                         // channels per wave
  constexpr int kWGC = 16 / kRPC;                        // channels per workgroup
  constexpr int kCSt = kRPC == 1 ? kCStride : kNS + 4;   // Cs step pitch (floats)
  constexpr int kNB = kRPC == 1 ? 2 : 1;                 // staging buffers
  const bool has_z = p.z != nullptr;
  const bool has_prez = !kPrep && p.out_prez != nullptr;
  float* const ck_out = p.ck;
  const bool has_ck = kPrep || ck_out != nullptr;
  float* const xs_out = p.chunk_states;
  // 4 rows per channel with 16-bit B / C (the reference's N = 64 benchmark
  // shape): B and C are staged at their storage width and each lane reads its
  // B values per 16-step block, so the kernel fits 3 waves per SIMD (159
  // VGPRs, 40 KB of LDS) instead of 2 (209, 56 KB); every value is converted
  // exactly, so the outputs keep their bits. At 2 rows per channel the fp32
  // staging already fits (39 KB) and the per-block B reads alone bring the
  // kernel to 3 waves per SIMD (150 VGPRs instead of 195); the 16-bit staging
  // would only add conversion work there.
  constexpr bool kH16 = kRPC == 4 && sizeof(TBC) == 2;
  constexpr int kB16P = kScanT + 8;  // halves per state row (144 bytes)
  constexpr int kC16P = kNS + 8;     // halves per step row
  __shared__ __align__(16) float Bs[kNB][kH16 ? 1 : kNS * kBStride];
  __shared__ __align__(16) float Cs[kNB][kH16 ? 1 : kScanT * kCSt];
  __shared__ __align__(16) uint16_t Bh[kH16 ? kNS * kB16P : 8];
  __shared__ __align__(16) uint16_t Ch[kH16 ? kScanT * kC16P : 8];
  __shared__ float hbuf[4][4 * kHC];

  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int c = lane / 16;       // row of the wave (the channel when kRPC == 1)
  const int n = lane % 16;       // lane in the row: owned step block / state
  const int sr = c % kRPC;       // row within the channel
  const int ns = 16 * sr + n;    // state owned by this lane

  const int per_batch = p.ngroups * p.tiles_per_group;
  const int b = blockIdx.x / per_batch;
  const int g = (blockIdx.x % per_batch) / p.tiles_per_group;
  const int tile = blockIdx.x % p.tiles_per_group;
  const int d0 = g * p.ch_per_group + tile * kWGC;      // first channel of the workgroup
  const int wc = wave * kCPW + c / kRPC;                // channel within the workgroup
  const int d = d0 + wc;
  const bool n_ok = ns < p.dstate;

  const float a_scaled = n_ok ? p.A[(int64_t)d * p.A_ds + ns] * kLog2e : 0.0f;
  const float dbias = p.delta_bias ? p.delta_bias[d] : 0.0f;
  const float dskip = p.D ? p.D[d] : 0.0f;

  // Wave-uniform resources over the workgroup's 16 channels (rows) and over
  // its group's B / C rows.
  const uint32_t L = (uint32_t)p.seqlen;
  auto row_rsrc = [&](const void* base, int64_t bs, int64_t ds, int esz) {
    const char* q = static_cast<const char*>(base) + ((int64_t)b * bs + (int64_t)d0 * ds) * esz;
    return make_rsrc(q, (uint32_t)(((kWGC - 1) * ds + L) * esz));
  };
  const Rsrc rs_u = row_rsrc(p.u, p.u_bs, p.u_ds, sizeof(TU));
  const Rsrc rs_d = row_rsrc(p.delta, p.d_bs, p.d_ds, sizeof(TD));
  const Rsrc rs_z = has_z ? row_rsrc(p.z, p.z_bs, p.z_ds, sizeof(TU)) : rs_u;
  const int64_t zds = has_z ? p.z_ds : p.u_ds;
  // the forward's output, or the preparation pass's dz (with a gate)
  const Rsrc rs_o = row_rsrc(kPrep ? p.dz : p.out, p.o_bs, p.o_ds, sizeof(TU));
  const Rsrc rs_oz = has_prez ? row_rsrc(p.out_prez, p.o_bs, p.o_ds, sizeof(TU)) : rs_o;
  const Rsrc rs_go = kPrep ? row_rsrc(p.dout, p.go_bs, p.go_ds, sizeof(TU)) : rs_u;
  const uint32_t vo_go1 = kPrep ? (uint32_t)(wc * p.go_ds + n) * sizeof(TU) : 0u;
  const uint32_t bc_bytes_B = (uint32_t)(((p.dstate - 1) * p.B_ns + L) * sizeof(TBC));
  const uint32_t bc_bytes_C = (uint32_t)(((p.dstate - 1) * p.C_ns + L) * sizeof(TBC));
  const Rsrc rs_B = make_rsrc(static_cast<const TBC*>(p.B) + (int64_t)b * p.B_bs + (int64_t)g * p.B_gs, bc_bytes_B);
  const Rsrc rs_C = make_rsrc(static_cast<const TBC*>(p.C) + (int64_t)b * p.C_bs + (int64_t)g * p.C_gs, bc_bytes_C);

  // Per-lane byte offsets, fixed for the whole scan.
  const uint32_t vo_d4 = (uint32_t)(wc * p.d_ds + 4 * n) * sizeof(TD);   // delta, steps 4n..4n+3
  const uint32_t vo_u4 = (uint32_t)(wc * p.u_ds + 4 * n) * sizeof(TU);   // u, steps 4n..4n+3
  const uint32_t vo_u1 = (uint32_t)(wc * p.u_ds + n) * sizeof(TU);       // u, step 16 blk + n
  const uint32_t vo_z1 = (uint32_t)(wc * zds + n) * sizeof(TU);
  const uint32_t vo_o1 = (uint32_t)(wc * p.o_ds + n) * sizeof(TU);
  // checkpoints [batch, nchunks, dim, dstate]: this batch's slab, the lane's
  // (channel, state) offset fixed, the chunk in the scalar offset
  const Rsrc rs_ck = make_rsrc(has_ck ? ck_out + (int64_t)b * p.nchunks * p.dim * p.dstate : p.A,
                               has_ck ? (uint32_t)((int64_t)p.nchunks * p.dim * p.dstate * 4) : 0u);
  const uint32_t vo_ck = (uint32_t)(d * p.dstate + ns) * 4u;
  const uint32_t ck_chunk_bytes = (uint32_t)(p.dim * p.dstate * 4);
  // staging: state sn, steps 4q..4q+3; the 16 lanes of a row take 16
  // different states, so the transposed Cs writes of a wave hit 64 distinct
  // banks (with 16 lanes per state they conflicted 8-way)
  const int sn = tid % 16, q = tid / 16;
  uint32_t vo_B[kRPC], vo_C[kRPC];  // state sn + 16 k
#pragma unroll
  for (int k = 0; k < kRPC; ++k) {
    const int sn_c = min(sn + 16 * k, p.dstate - 1);
    vo_B[k] = (uint32_t)(sn_c * p.B_ns + 4 * q) * sizeof(TBC);
    vo_C[k] = (uint32_t)(sn_c * p.C_ns + 4 * q) * sizeof(TBC);
  }

  struct Regs {
    Raw4<TD> dv;
    Raw4<TU> uv;
    Raw1<TU> uo[4], zo[4];
    Raw1<TU> go[kPrep ? 4 : 1];
  };
  struct Stage {
    Raw4<TBC> bv[kRPC], cv[kRPC];
  };
  const int nt = p.seqlen / kScanT;
  auto load_regs = [&](int t, Regs& r) {
    const uint32_t l0 = (uint32_t)t * kScanT;
    r.dv = bload4<TD>(rs_d, vo_d4, l0 * sizeof(TD));
    r.uv = bload4<TU>(rs_u, vo_u4, l0 * sizeof(TU));
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      r.uo[blk] = bload1<TU>(rs_u, vo_u1 + 16 * blk * sizeof(TU), l0 * sizeof(TU));
      r.zo[blk] = bload1<TU>(rs_z, vo_z1 + 16 * blk * sizeof(TU), l0 * sizeof(TU));
      if constexpr (kPrep) r.go[blk] = bload1<TU>(rs_go, vo_go1 + 16 * blk * sizeof(TU), l0 * sizeof(TU));
    }
  };
  auto load_stage = [&](int t, Stage& s) {
    const uint32_t l0 = (uint32_t)t * kScanT;
#pragma unroll
    for (int k = 0; k < kRPC; ++k) {
      s.bv[k] = bload4<TBC>(rs_B, vo_B[k], l0 * sizeof(TBC));
      s.cv[k] = bload4<TBC>(rs_C, vo_C[k], l0 * sizeof(TBC));
    }
  };
  auto write_stage = [&](const Stage& s, int buf) {
#pragma unroll
    for (int kk = 0; kk < kRPC; ++kk) {
      const int st = sn + 16 * kk;
      const bool ok = st < p.dstate;
      if constexpr (kH16) {
        const u32x2 bw = (u32x2)s.bv[kk];
        *reinterpret_cast<u32x2*>(&Bh[st * kB16P + 4 * q]) = ok ? bw : (u32x2){0u, 0u};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t w = s.cv[kk][k >> 1];
          Ch[(4 * q + k) * kC16P + st] = ok ? (uint16_t)((k & 1) ? (w >> 16) : (w & 0xFFFFu)) : (uint16_t)0;
        }
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          Bs[buf][st * kBStride + 4 * q + k] = ok ? raw4_f32<TBC>(s.bv[kk], k) : 0.0f;
          Cs[buf][(4 * q + k) * kCSt + st] = ok ? raw4_f32<TBC>(s.cv[kk], k) : 0.0f;
        }
      }
    }
  };

  float h = 0.0f;
  float* hb = hbuf[wave];
  float ph[16] = {}, pc[16] = {};  // pending block: h[c][j][0..15] and C[j][0..15]
  float p_uo = 0.0f, p_zo = 0.0f, p_go = 0.0f;
  uint32_t p_off = 0;     // byte offset of the pending output element
  bool pending = false;   // wave-uniform
  auto finish_pending = [&]() {
    float y4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 16; ++s) y4[s & 3] = fmaf(ph[s], pc[s], y4[s & 3]);
    float ysum = (y4[0] + y4[1]) + (y4[2] + y4[3]);
    // rows of one channel: add their partial sums (every row gets the total)
    if constexpr (kRPC == 4) ysum = swap32_sum(ysum, ysum);
    if constexpr (kRPC >= 2) ysum = swap16_sum(ysum, ysum);
    if (kRPC > 1 && sr != 0) return;  // the channel's first row stores
    float o = fmaf(dskip, p_uo, ysum);
    if constexpr (kPrep) {
      if (has_z) {
        const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-p_zo * kLog2e));
        bstore1<TU>(rs_o, p_off, p_go * o * sg * fmaf(p_zo, 1.0f - sg, 1.0f));
      }
    } else {
      if (has_prez) bstore1<TU>(rs_oz, p_off, o);
      if (has_z) o *= silu_fast(p_zo);
      bstore1<TU>(rs_o, p_off, o);
    }
  };
  float dsum = 0.0f;  // sum of delta' since step 0 (chunk states)

  auto compute = [&](int t, const Regs& cur) {
    const int buf = t & 1;
    float hck[kScanT / 16];  // the states before the tile's 16-step blocks (checkpoints)
    float dl[4], du[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float dv = raw4_f32<TD>(cur.dv, k) + dbias;
      if constexpr (kSoftplus) dv = softplus_f32(dv);
      dl[k] = dv;
      du[k] = dv * raw4_f32<TU>(cur.uv, k);
    }
    // wait states between the last VALU write of dl / du and their DPP reads
    asm volatile("s_nop 1"
                 : "+v"(dl[0]), "+v"(dl[1]), "+v"(dl[2]), "+v"(dl[3]), "+v"(du[0]), "+v"(du[1]),
                   "+v"(du[2]), "+v"(du[3]));
    const int bb = kNB == 2 ? buf : 0;
    constexpr bool kBBlk = kH16 || kRPC == 2;  // B read per 16-step block
    float bt[kBBlk ? 16 : kScanT];
    if constexpr (!kBBlk) {
#pragma unroll
      for (int l = 0; l < kScanT; ++l) bt[l] = Bs[bb][ns * kBStride + l];
    }

#pragma unroll
    for (int blk = 0; blk < kScanT / 16; ++blk) {
      hck[blk] = h;
      if constexpr (kBBlk) {
        if constexpr (kH16) {
          const u32x4* src = reinterpret_cast<const u32x4*>(&Bh[ns * kB16P + 16 * blk]);
          const u32x4 w0 = src[0], w1 = src[1];
#pragma unroll
          for (int l = 0; l < 8; ++l) {
            const uint32_t w = l < 4 ? w0[l] : w1[l - 4];
            bt[2 * l] = raw_f32<TBC>((uint16_t)(w & 0xFFFFu));
            bt[2 * l + 1] = raw_f32<TBC>((uint16_t)(w >> 16));
          }
        } else {
#pragma unroll
          for (int l = 0; l < 16; ++l) bt[l] = Bs[bb][ns * kBStride + 16 * blk + l];
        }
      }
      float hv[16], av[16], xv[16];
      auto steps4 = [&](auto src_c, int j4) {
        constexpr int kSrc = decltype(src_c)::value;
#pragma unroll
        for (int k = 0; k < 4; ++k) av[4 * j4 + k] = mul_bcast<kSrc>(dl[k], a_scaled);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          xv[4 * j4 + k] = mul_bcast<kSrc>(du[k], bt[(kBBlk ? 0 : 16 * blk) + 4 * j4 + k]);
      };
      switch (blk) {
        case 0:
          steps4(std::integral_constant<int, 0>{}, 0); steps4(std::integral_constant<int, 1>{}, 1);
          steps4(std::integral_constant<int, 2>{}, 2); steps4(std::integral_constant<int, 3>{}, 3);
          break;
        case 1:
          steps4(std::integral_constant<int, 4>{}, 0); steps4(std::integral_constant<int, 5>{}, 1);
          steps4(std::integral_constant<int, 6>{}, 2); steps4(std::integral_constant<int, 7>{}, 3);
          break;
        case 2:
          steps4(std::integral_constant<int, 8>{}, 0); steps4(std::integral_constant<int, 9>{}, 1);
          steps4(std::integral_constant<int, 10>{}, 2); steps4(std::integral_constant<int, 11>{}, 3);
          break;
        default:
          steps4(std::integral_constant<int, 12>{}, 0); steps4(std::integral_constant<int, 13>{}, 1);
          steps4(std::integral_constant<int, 14>{}, 2); steps4(std::integral_constant<int, 15>{}, 3);
          break;
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) av[j] = __builtin_amdgcn_exp2f(av[j]);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        h = fmaf(av[j], h, xv[j]);
        hv[j] = h;
      }
      asm volatile("" : "+v"(h));
      __builtin_amdgcn_sched_barrier(0);
      if (pending) finish_pending();  // previous block's output
#pragma unroll
      for (int j = 0; j < 16; ++j) hb[c * kHC + j * kHJ + n] = hv[j];
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int s2 = 0; s2 < 16; ++s2) ph[s2] = hb[c * kHC + n * kHJ + s2];
      if constexpr (kH16) {
        const u32x4* src = reinterpret_cast<const u32x4*>(&Ch[(16 * blk + n) * kC16P + 16 * sr]);
        const u32x4 w0 = src[0], w1 = src[1];
#pragma unroll
        for (int l = 0; l < 8; ++l) {
          const uint32_t w = l < 4 ? w0[l] : w1[l - 4];
          pc[2 * l] = raw_f32<TBC>((uint16_t)(w & 0xFFFFu));
          pc[2 * l + 1] = raw_f32<TBC>((uint16_t)(w >> 16));
        }
      } else {
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2) pc[s2] = Cs[bb][(16 * blk + n) * kCSt + 16 * sr + s2];
      }
      __builtin_amdgcn_wave_barrier();
      p_uo = raw_f32<TU>(cur.uo[blk]);
      p_zo = has_z ? raw_f32<TU>(cur.zo[blk]) : 0.0f;
      if constexpr (kPrep) p_go = raw_f32<TU>(cur.go[blk]);
      p_off = vo_o1 + ((uint32_t)t * kScanT + 16 * blk) * sizeof(TU);
      pending = true;
    }
    // the tile's checkpoints in one burst after its last block (stored before
    // each block they cost about 6 us more at the C5 shape)
    if (has_ck && n_ok) {
#pragma unroll
      for (int blk = 0; blk < kScanT / 16; ++blk)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, hck[blk]), rs_ck, (int)vo_ck,
                                              (int)((uint32_t)((t * kScanT + 16 * blk) / kCk) * ck_chunk_bytes), 0);
    }
    if (!kPrep && xs_out) {
      dsum += row16_sum((dl[0] + dl[1]) + (dl[2] + dl[3]));
      const int l1 = (t + 1) * kScanT;
      if ((l1 % kXChunk == 0 || l1 >= p.seqlen) && n_ok) {
        float* xs = xs_out +
                    ((((int64_t)b * p.dim + d) * p.xchunks + (l1 - 1) / kXChunk) * p.dstate + ns) * 2;
        xs[0] = __builtin_amdgcn_exp2f(a_scaled * dsum);
        xs[1] = h;
      }
    }
  };

  // One tile: publish tile t's staging (barrier), stage tile t + 1, issue
  // the loads of tile t + 2's B / C and tile t + 1's delta / u / z (clamped
  // to the last tile: unconditional loads of valid addresses), then compute.
  Stage st;
  auto tile_body = [&](int t, const Regs& cur, Regs& nxt) {
    if constexpr (kNB == 2) {
      __syncthreads();
      write_stage(st, (t + 1) & 1);
      load_stage(min(t + 2, nt - 1), st);
    } else {
      // single buffer: tile t's stage (in st since the previous tile) goes in
      // once every wave is done with tile t - 1's
      __syncthreads();
      write_stage(st, 0);
      __syncthreads();
      load_stage(min(t + 1, nt - 1), st);
    }
    load_regs(min(t + 1, nt - 1), nxt);
    asm volatile("" ::: "memory");
    compute(t, cur);
  };

  Regs ra, rb;
  load_stage(0, st);
  load_regs(0, ra);
  if constexpr (kNB == 2) {
    write_stage(st, 0);
    load_stage(min(1, nt - 1), st);
  }
  for (int t = 0; t < nt; t += 2) {
    tile_body(t, ra, rb);
    if (t + 1 < nt) tile_body(t + 1, rb, ra);
  }
  finish_pending();
  if (!kPrep && p.last_state && n_ok) {
    p.last_state[((int64_t)b * p.dim + d) * p.dstate + ns] = h;
  }
}

// ---------------------------------------------------------------------------
// Producer / consumer split of the whole-tile forward for dstate <= 16
// (mamba_scan_split_kernel). At the C5 shape the (channel, state) lanes fill
// only 2 waves per SIMD, and at that occupancy the recurrence's dependent FMA
// chain and exp2 latency leave the SIMDs idle about a third of the time. This
// kernel doubles the waves without duplicating any arithmetic: a workgroup of
// 16 channels has 8 waves. Waves 0-3 (producers) run the recurrence exactly as
// mamba_scan_fast_kernel does and write each 16-step block's states into a
// transpose buffer; waves 4-7 (consumers) read block K's states while the
// producers compute block K + 1, and form the outputs: y = sum_n h C + D u,
// then the gate, or in the backward's preparation pass dz. The transpose
// buffer is double-buffered per producer wave and one workgroup barrier per
// block hands it over (LDS counters between each producer / consumer pair
// instead measured 9-20% slower: the flag round trips sit on the producers'
// critical path). Producers run at a raised wave priority (s_setprio 2), so a
// SIMD issues the recurrence first and fills its gaps with consumer work. The
// producers stage B, the consumers C, each double-buffered per 64-step tile.
// The arithmetic and its order are those of mamba_scan_fast_kernel, so every
// output has the same bits.
//
// kMode: kFwdLean / kFwdTrain as for mamba_scan_fast_kernel (a gate z is
// required); kFwdAny: any forward, the gate, pre-gate output, checkpoints and
// chunk states tested at run time (the compiled binding's fwd, which returns
// the chunk states); or kPrepGated: the backward's preparation pass with a
// gate (checkpoints by the producers, dz = dout y sigma(z) (1 + z (1 -
// sigma(z))) by the consumers).
enum { kPrepGated = 3 };

template <typename TU, typename TD, typename TBC, bool kSoftplus, int kMode>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4)))
mamba_scan_split_kernel(ScanParams p) {
  constexpr bool kPrep = kMode == kPrepGated;
  const bool has_z = kMode != kFwdAny || p.z != nullptr;
  const bool has_prez = kMode == kFwdTrain || (kMode == kFwdAny && p.out_prez != nullptr);
  const bool has_ck = kMode == kFwdTrain || kPrep || (kMode == kFwdAny && p.ck != nullptr);
  float* const xs_out = kMode == kFwdAny ? p.chunk_states : nullptr;
  __shared__ float Bs[2][16 * kBStride];
  __shared__ float Cs[2][kScanT * kCStride];
  __shared__ float hbuf[2][4][4 * kHC];  // [block parity][producer wave][c][j][n]

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);  // wave-uniform role
  const bool producer = wave < 4;
  const int pw = wave & 3;  // the producer / consumer pair: channels 4 pw .. 4 pw + 3
  const int lane = tid % 64;
  const int c = lane / 16;
  const int n = lane % 16;
  const int per_batch = p.ngroups * p.tiles_per_group;
  const int b = blockIdx.x / per_batch;
  const int g = (blockIdx.x % per_batch) / p.tiles_per_group;
  const int tile = blockIdx.x % p.tiles_per_group;
  const int d0 = g * p.ch_per_group + tile * kScanCh;
  const int wc = pw * 4 + c;
  const int d = d0 + wc;
  const bool n_ok = n < p.dstate;
  const uint32_t L = (uint32_t)p.seqlen;
  const int nt = p.seqlen / kScanT;
  auto row_rsrc = [&](const void* base, int64_t bs, int64_t ds, int esz) {
    const char* q = static_cast<const char*>(base) + ((int64_t)b * bs + (int64_t)d0 * ds) * esz;
    return make_rsrc(q, (uint32_t)(((kScanCh - 1) * ds + L) * esz));
  };
  // staging: thread r of each role loads state sn, steps 4 q .. 4 q + 3 of B
  // (producers) or C (consumers)
  const int r = tid & 255;
  const int sn = r % 16, q = r / 16;
  const int sn_c = min(sn, p.dstate - 1);
  const bool s_ok = sn < p.dstate;

  if (producer) {
    __builtin_amdgcn_s_setprio(2);
    const float a_scaled = n_ok ? p.A[(int64_t)d * p.A_ds + n] * kLog2e : 0.0f;
    const float dbias = p.delta_bias ? p.delta_bias[d] : 0.0f;
    const Rsrc rs_u = row_rsrc(p.u, p.u_bs, p.u_ds, sizeof(TU));
    const Rsrc rs_d = row_rsrc(p.delta, p.d_bs, p.d_ds, sizeof(TD));
    const uint32_t bc_bytes_B = (uint32_t)(((p.dstate - 1) * p.B_ns + L) * sizeof(TBC));
    const Rsrc rs_B = make_rsrc(static_cast<const TBC*>(p.B) + (int64_t)b * p.B_bs + (int64_t)g * p.B_gs, bc_bytes_B);
    const uint32_t vo_d4 = (uint32_t)(wc * p.d_ds + 4 * n) * sizeof(TD);  // delta, steps 4n..4n+3
    const uint32_t vo_u4 = (uint32_t)(wc * p.u_ds + 4 * n) * sizeof(TU);
    const uint32_t vo_B = (uint32_t)(sn_c * p.B_ns + 4 * q) * sizeof(TBC);
    // checkpoints [batch, nchunks, dim, dstate]: the batch's slab, the chunk in the scalar offset
    const Rsrc rs_ck = make_rsrc(has_ck ? p.ck + (int64_t)b * p.nchunks * p.dim * p.dstate : p.A,
                                 has_ck ? (uint32_t)((int64_t)p.nchunks * p.dim * p.dstate * 4) : 0u);
    const uint32_t vo_ck = (uint32_t)(d * p.dstate + n) * 4u;
    const uint32_t ck_chunk_bytes = (uint32_t)(p.dim * p.dstate * 4);
    struct Regs {
      Raw4<TD> dv;
      Raw4<TU> uv;
    };
    auto load_regs = [&](int t, Regs& rr) {
      const uint32_t l0 = (uint32_t)t * kScanT;
      rr.dv = bload4<TD>(rs_d, vo_d4, l0 * sizeof(TD));
      rr.uv = bload4<TU>(rs_u, vo_u4, l0 * sizeof(TU));
    };
    auto write_B = [&](const Raw4<TBC>& v, int buf) {
#pragma unroll
      for (int k = 0; k < 4; ++k) Bs[buf][sn * kBStride + 4 * q + k] = s_ok ? raw4_f32<TBC>(v, k) : 0.0f;
    };
    Raw4<TBC> sv = bload4<TBC>(rs_B, vo_B, 0u);
    Regs ra, rb;
    load_regs(0, ra);
    write_B(sv, 0);
    sv = bload4<TBC>(rs_B, vo_B, (uint32_t)min(1, nt - 1) * kScanT * sizeof(TBC));
    __syncthreads();
    float h = 0.0f;
    float dsum = 0.0f;  // sum of delta' since step 0 (chunk states)
    // Tile t: stage tile t + 1's B (its buffer was last read in tile t - 1,
    // before the barrier that ended it), issue the loads of tile t + 2's B
    // and tile t + 1's delta / u (clamped to the last tile), then the four
    // blocks, each ending with the states written and a barrier.
    auto tile_body = [&](int t, const Regs& cur, Regs& nxt) {
      write_B(sv, (t + 1) & 1);
      sv = bload4<TBC>(rs_B, vo_B, (uint32_t)min(t + 2, nt - 1) * kScanT * sizeof(TBC));
      load_regs(min(t + 1, nt - 1), nxt);
      asm volatile("" ::: "memory");
      const int buf = t & 1;
      float hck[kScanT / 16];  // the states before the tile's 16-step blocks (checkpoints)
      float dl[4], du[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float dv = raw4_f32<TD>(cur.dv, k) + dbias;
        if constexpr (kSoftplus) dv = softplus_f32(dv);
        dl[k] = dv;
        du[k] = dv * raw4_f32<TU>(cur.uv, k);
      }
      // wait states between the last VALU write of dl / du and their DPP reads
      asm volatile("s_nop 1"
                   : "+v"(dl[0]), "+v"(dl[1]), "+v"(dl[2]), "+v"(dl[3]), "+v"(du[0]), "+v"(du[1]),
                     "+v"(du[2]), "+v"(du[3]));
#pragma unroll
      for (int blk = 0; blk < kScanT / 16; ++blk) {
        hck[blk] = h;
        float bt[16], hv[16], av[16], xv[16];
#pragma unroll
        for (int l = 0; l < 16; ++l) bt[l] = Bs[buf][n * kBStride + 16 * blk + l];
        auto steps4 = [&](auto src_c, int j4) {
          constexpr int kSrc = decltype(src_c)::value;
#pragma unroll
          for (int k = 0; k < 4; ++k) av[4 * j4 + k] = mul_bcast<kSrc>(dl[k], a_scaled);
#pragma unroll
          for (int k = 0; k < 4; ++k) xv[4 * j4 + k] = mul_bcast<kSrc>(du[k], bt[4 * j4 + k]);
        };
        switch (blk) {
          case 0:
            steps4(std::integral_constant<int, 0>{}, 0); steps4(std::integral_constant<int, 1>{}, 1);
            steps4(std::integral_constant<int, 2>{}, 2); steps4(std::integral_constant<int, 3>{}, 3);
            break;
          case 1:
            steps4(std::integral_constant<int, 4>{}, 0); steps4(std::integral_constant<int, 5>{}, 1);
            steps4(std::integral_constant<int, 6>{}, 2); steps4(std::integral_constant<int, 7>{}, 3);
            break;
          case 2:
            steps4(std::integral_constant<int, 8>{}, 0); steps4(std::integral_constant<int, 9>{}, 1);
            steps4(std::integral_constant<int, 10>{}, 2); steps4(std::integral_constant<int, 11>{}, 3);
            break;
          default:
            steps4(std::integral_constant<int, 12>{}, 0); steps4(std::integral_constant<int, 13>{}, 1);
            steps4(std::integral_constant<int, 14>{}, 2); steps4(std::integral_constant<int, 15>{}, 3);
            break;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) av[j] = __builtin_amdgcn_exp2f(av[j]);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          h = fmaf(av[j], h, xv[j]);
          hv[j] = h;
        }
        // block 4 t + blk's states, [c][j][n]: its buffer was last read (block
        // 4 t + blk - 2) before the previous barrier
        float* hb = hbuf[blk & 1][pw];
#pragma unroll
        for (int j = 0; j < 16; ++j) hb[c * kHC + j * kHJ + n] = hv[j];
        __syncthreads();
      }
      if (has_ck && n_ok) {
#pragma unroll
        for (int blk = 0; blk < kScanT / 16; ++blk)
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, hck[blk]), rs_ck, (int)vo_ck,
                                                (int)((uint32_t)((t * kScanT + 16 * blk) / kCk) * ck_chunk_bytes), 0);
      }
      if (xs_out) {
        // the channel's delta' over the tile, then (decay product, state) at
        // each 2048-step chunk end
        dsum += row16_sum((dl[0] + dl[1]) + (dl[2] + dl[3]));
        const int l1 = (t + 1) * kScanT;
        if ((l1 % kXChunk == 0 || l1 >= p.seqlen) && n_ok) {
          float* xs = xs_out + ((((int64_t)b * p.dim + d) * p.xchunks + (l1 - 1) / kXChunk) * p.dstate + n) * 2;
          xs[0] = __builtin_amdgcn_exp2f(a_scaled * dsum);
          xs[1] = h;
        }
      }
    };
    for (int t = 0; t < nt; t += 2) {
      tile_body(t, ra, rb);
      if (t + 1 < nt) tile_body(t + 1, rb, ra);
    }
    if (!kPrep && p.last_state && n_ok) p.last_state[((int64_t)b * p.dim + d) * p.dstate + n] = h;
  } else {
    const float dskip = p.D ? p.D[d] : 0.0f;
    const Rsrc rs_u = row_rsrc(p.u, p.u_bs, p.u_ds, sizeof(TU));
    // without a gate the z loads read u again (valid addresses, unused)
    const Rsrc rs_z = has_z ? row_rsrc(p.z, p.z_bs, p.z_ds, sizeof(TU)) : rs_u;
    const int64_t zds = has_z ? p.z_ds : p.u_ds;
    // the forward's output, or the preparation pass's dz
    const Rsrc rs_o = row_rsrc(kPrep ? p.dz : p.out, p.o_bs, p.o_ds, sizeof(TU));
    const Rsrc rs_oz = has_prez ? row_rsrc(p.out_prez, p.o_bs, p.o_ds, sizeof(TU)) : rs_o;
    const Rsrc rs_go = kPrep ? row_rsrc(p.dout, p.go_bs, p.go_ds, sizeof(TU)) : rs_u;
    const uint32_t bc_bytes_C = (uint32_t)(((p.dstate - 1) * p.C_ns + L) * sizeof(TBC));
    const Rsrc rs_C = make_rsrc(static_cast<const TBC*>(p.C) + (int64_t)b * p.C_bs + (int64_t)g * p.C_gs, bc_bytes_C);
    // lane (c, n) forms step 16 blk + n of channel wc
    const uint32_t vo_u1 = (uint32_t)(wc * p.u_ds + n) * sizeof(TU);
    const uint32_t vo_z1 = (uint32_t)(wc * zds + n) * sizeof(TU);
    const uint32_t vo_o1 = (uint32_t)(wc * p.o_ds + n) * sizeof(TU);
    const uint32_t vo_go1 = kPrep ? (uint32_t)(wc * p.go_ds + n) * sizeof(TU) : 0u;
    const uint32_t vo_C = (uint32_t)(sn_c * p.C_ns + 4 * q) * sizeof(TBC);
    struct Regs {
      Raw1<TU> uo[4], zo[4];
      Raw1<TU> go[kPrep ? 4 : 1];
    };
    auto load_regs = [&](int t, Regs& rr) {
      const uint32_t l0 = (uint32_t)t * kScanT;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        rr.uo[blk] = bload1<TU>(rs_u, vo_u1 + 16 * blk * sizeof(TU), l0 * sizeof(TU));
        rr.zo[blk] = bload1<TU>(rs_z, vo_z1 + 16 * blk * sizeof(TU), l0 * sizeof(TU));
        if constexpr (kPrep) rr.go[blk] = bload1<TU>(rs_go, vo_go1 + 16 * blk * sizeof(TU), l0 * sizeof(TU));
      }
    };
    auto write_C = [&](const Raw4<TBC>& v, int buf) {
#pragma unroll
      for (int k = 0; k < 4; ++k) Cs[buf][(4 * q + k) * kCStride + sn] = s_ok ? raw4_f32<TBC>(v, k) : 0.0f;
    };
    Raw4<TBC> sv = bload4<TBC>(rs_C, vo_C, 0u);
    Regs ra, rb;
    load_regs(0, ra);
    write_C(sv, 0);
    sv = bload4<TBC>(rs_C, vo_C, (uint32_t)min(1, nt - 1) * kScanT * sizeof(TBC));
    __syncthreads();
    // Tile t: after each block's barrier, that block's states are complete;
    // after the first, stage tile t + 1's C (its buffer was last read for
    // block 4 t - 1, before that barrier) and issue the next loads.
    auto tile_body = [&](int t, const Regs& cur, Regs& nxt) {
      const int buf = t & 1;
#pragma unroll
      for (int blk = 0; blk < kScanT / 16; ++blk) {
        __syncthreads();
        if (blk == 0) {
          write_C(sv, (t + 1) & 1);
          sv = bload4<TBC>(rs_C, vo_C, (uint32_t)min(t + 2, nt - 1) * kScanT * sizeof(TBC));
          load_regs(min(t + 1, nt - 1), nxt);
          asm volatile("" ::: "memory");
        }
        const float* hb = hbuf[blk & 1][pw];
        float ph[16], pc[16];
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2) {
          ph[s2] = hb[c * kHC + n * kHJ + s2];
          pc[s2] = Cs[buf][(16 * blk + n) * kCStride + s2];
        }
        float y4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 16; ++s) y4[s & 3] = fmaf(ph[s], pc[s], y4[s & 3]);
        const float ysum = (y4[0] + y4[1]) + (y4[2] + y4[3]);
        // each stored value is rounded to fp32 and then to the storage type, as
        // the single-role kernel and the reference do: the opaque copies keep
        // the compiler from fusing the last FMA or product with an fp16
        // conversion (v_fma_mixlo_f16, one rounding)
        float o = fmaf(dskip, raw_f32<TU>(cur.uo[blk]), ysum);
        asm("" : "+v"(o));
        const float zv = raw_f32<TU>(cur.zo[blk]);
        const uint32_t off = vo_o1 + ((uint32_t)t * kScanT + 16 * blk) * sizeof(TU);
        float v;
        if constexpr (kPrep) {
          const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-zv * kLog2e));
          v = raw_f32<TU>(cur.go[blk]) * o * sg * fmaf(zv, 1.0f - sg, 1.0f);
        } else {
          if (has_prez) bstore1<TU>(rs_oz, off, o);
          v = has_z ? o * silu_fast(zv) : o;
        }
        asm("" : "+v"(v));
        bstore1<TU>(rs_o, off, v);
      }
    };
    for (int t = 0; t < nt; t += 2) {
      tile_body(t, ra, rb);
      if (t + 1 < nt) tile_body(t + 1, rb, ra);
    }
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

// The same recurrence in chunks of lc steps, for shapes whose (batch, channel)
// lanes are too few to keep the GPU busy (AMADEUS: 384 channels; the
// sequential kernel above then runs at about 6% of HBM bandwidth). Three
// launches, lanes (batch, chunk, channel) with channels coalesced, and the
// output buffer as the only scratch:
//   1. every chunk but the last: its decay product P = prod dA and its state
//      from zero S, stored in the first two rows of the chunk in y;
//   2. per (batch, channel), sequentially over the chunks: the state entering
//      chunk k, s_k = P_{k-1} s_{k-1} + S_{k-1}, stored over P_k (the row a
//      chunk's own lane reads before writing anything);
//   3. every chunk from its entering state: s = dA s + dBx, y = C s + D x.
// 8 bytes per element more than the sequential pass (dA and dBx read twice);
// the states differ from the sequential ones by rounding only. Chunks: see
// diag_chunks.
template <int kLC>
__global__ void __launch_bounds__(256)
diag_scan_chunk_agg_kernel(const float* __restrict__ dA, const float* __restrict__ dBx,
                           float* __restrict__ y, int batch, int seqlen, int d_inner, int lc,
                           int nchunks) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_b = (int64_t)(nchunks - 1) * d_inner;
  if (gid >= (int64_t)batch * per_b) return;
  const int b = (int)(gid / per_b);
  const int k = (int)((gid % per_b) / d_inner);
  const int d = (int)(gid % d_inner);
  const int64_t row0 = (int64_t)b * seqlen + (int64_t)k * lc;
  int64_t idx = row0 * d_inner + d;
  float P = 1.0f, S = 0.0f;
  if constexpr (kLC > 0) {
    // a full chunk (lc <= kLC steps), its rows loaded together
    float a[kLC], v[kLC];
#pragma unroll
    for (int t = 0; t < kLC; ++t) {
      const bool in = t < lc;
      const int64_t i = idx + (int64_t)(in ? t : 0) * d_inner;
      a[t] = in ? dA[i] : 1.0f;
      v[t] = in ? dBx[i] : 0.0f;
    }
#pragma unroll
    for (int t = 0; t < kLC; ++t) {
      S = fmaf(a[t], S, v[t]);
      P *= a[t];
    }
  } else {
#pragma unroll 8
    for (int t = 0; t < lc; ++t, idx += d_inner) {
      const float a = dA[idx];
      S = fmaf(a, S, dBx[idx]);
      P *= a;
    }
  }
  y[row0 * d_inner + d] = P;
  y[(row0 + 1) * d_inner + d] = S;
}

__global__ void __launch_bounds__(256)
diag_scan_chunk_carry_kernel(float* __restrict__ y, int batch, int seqlen, int d_inner, int lc,
                             int nchunks) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)batch * d_inner) return;
  const int b = (int)(gid / d_inner);
  const int d = (int)(gid % d_inner);
  // the aggregates of up to 16 chunks are loaded before any of their rows is
  // overwritten, so the loads do not wait on the chain
  constexpr int kG = 16;
  float s = 0.0f;
  const int64_t base = (int64_t)b * seqlen * d_inner + d;
  const int64_t chunk_stride = (int64_t)lc * d_inner;
  for (int k0 = 0; k0 + 1 < nchunks; k0 += kG) {
    float P[kG], S[kG];
#pragma unroll
    for (int i = 0; i < kG; ++i) {
      const int k = min(k0 + i, nchunks - 2);
      P[i] = y[base + k * chunk_stride];
      S[i] = y[base + k * chunk_stride + d_inner];
    }
#pragma unroll
    for (int i = 0; i < kG; ++i) {
      if (k0 + i + 1 < nchunks) {
        y[base + (k0 + i) * chunk_stride] = s;  // the state entering chunk k0 + i
        s = fmaf(P[i], s, S[i]);
      }
    }
  }
  y[base + (int64_t)(nchunks - 1) * chunk_stride] = s;
}

// Chunks for the diagonal scan: enough for about 2^lanes_log2 lanes in all,
// at most 64, at least 16 steps each; 1 means the sequential kernels. Both
// directions aim at 2^18 lanes; chunks of at most 32 steps are held in
// registers. The backward falls back to 2^17 for chunks that stream (at
// AMADEUS's shape [16, 1024, 384], streaming: backward 124 against 137 us
// with 2^19; registers: 43 chunks of 24 steps ran 1-2% faster than 64 of 16
// in both directions).
inline int diag_chunks(int64_t batch, int64_t seqlen, int64_t d_inner, int lanes_log2) {
  const int64_t lanes = batch * d_inner;
  const int64_t want = ((int64_t)1 << lanes_log2);
  int64_t nchunks = lanes >= want ? 1 : (want + lanes - 1) / lanes;
  nchunks = std::min<int64_t>(std::min<int64_t>(nchunks, 64), seqlen / 16);
  return (int)std::max<int64_t>(nchunks, 1);
}

template <int kLC>
__global__ void __launch_bounds__(256)
diag_scan_chunk_out_kernel(const float* __restrict__ dA, const float* __restrict__ dBx,
                           const float* __restrict__ C, const float* __restrict__ D,
                           const float* __restrict__ x, float* __restrict__ y, int batch,
                           int seqlen, int d_inner, int lc, int nchunks) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_b = (int64_t)nchunks * d_inner;
  if (gid >= (int64_t)batch * per_b) return;
  const int b = (int)(gid / per_b);
  const int k = (int)((gid % per_b) / d_inner);
  const int d = (int)(gid % d_inner);
  const int t0 = k * lc;
  const int n = min(lc, seqlen - t0);
  int64_t idx = ((int64_t)b * seqlen + t0) * d_inner + d;
  float s = y[idx];  // the entering state, read before this lane writes its rows
  const float dd = D[d];
  if constexpr (kLC > 0) {
    // the chunk's rows (at most kLC) loaded together
    float a[kLC], v[kLC], c[kLC], xv[kLC];
#pragma unroll
    for (int t = 0; t < kLC; ++t) {
      const bool in = t < n;
      const int64_t i = idx + (int64_t)(in ? t : 0) * d_inner;
      a[t] = in ? dA[i] : 1.0f;
      v[t] = in ? dBx[i] : 0.0f;
      c[t] = in ? C[i] : 0.0f;
      xv[t] = in ? x[i] : 0.0f;
    }
#pragma unroll
    for (int t = 0; t < kLC; ++t) {
      s = fmaf(a[t], s, v[t]);
      if (t < n) y[idx + (int64_t)t * d_inner] = fmaf(c[t], s, dd * xv[t]);
    }
  } else {
#pragma unroll 8
    for (int t = 0; t < n; ++t, idx += d_inner) {
      s = fmaf(dA[idx], s, dBx[idx]);
      y[idx] = fmaf(C[idx], s, dd * x[idx]);
    }
  }
}

// One launch for the whole forward when the sequence has at most 1024 steps
// and the (batch, channel) lanes are few: a workgroup takes 32 channels of
// one batch row (128-byte row segments) and cuts the sequence into nck
// chunks of at most 32 steps, one thread per (chunk, channel). Each thread
// holds its chunk's dA and dBx in registers and forms the chunk's decay
// product P and state from zero S; the chunks' (P, S) meet in LDS, where one
// thread per channel walks them in order (s_k = P_{k-1} s_{k-1} + S_{k-1}),
// and every thread then runs its rows from its entering state, reading C and
// x in two halves. Inputs are read once and y written once, with no scratch
// in HBM; the states differ from the sequential ones by rounding only.
// (Loading the first half during the carry, or C and x in four groups of 8
// rows one group ahead, measured 1% and 17% slower.)
constexpr int kDiagWgCh = 32;  // channels per workgroup
constexpr int kDiagWgLC = 32;  // steps per chunk at most (and chunks at most)

// 32-bit byte offsets from an array's base (the workgroup paths require
// batch * seqlen * d_inner * 4 < 2^32): the base stays in scalar registers
// and one offset register per row serves every array.
__device__ __forceinline__ float ld_at(const float* __restrict__ p, uint32_t e) {
  return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(p) + 4u * e);
}
__device__ __forceinline__ void st_at(float* __restrict__ p, uint32_t e, float v) {
  *reinterpret_cast<float*>(reinterpret_cast<char*>(p) + 4u * e) = v;
}

__global__ void __launch_bounds__(1024)
diag_scan_wg_kernel(const float* __restrict__ dA, const float* __restrict__ dBx,
                    const float* __restrict__ C, const float* __restrict__ D,
                    const float* __restrict__ x, float* __restrict__ y, int batch, int seqlen,
                    int d_inner, int lc, int nck) {
  __shared__ float sP[kDiagWgLC][kDiagWgCh + 1], sS[kDiagWgLC][kDiagWgCh + 1];
  const int c = threadIdx.x % kDiagWgCh;
  const int k = threadIdx.x / kDiagWgCh;  // chunk (< nck <= 32)
  const int dblocks = (d_inner + kDiagWgCh - 1) / kDiagWgCh;
  const int b = blockIdx.x / dblocks;
  const int d = (blockIdx.x % dblocks) * kDiagWgCh + c;
  const bool live = d < d_inner;
  const int t0 = k * lc;
  const int n = live ? max(0, min(lc, seqlen - t0)) : 0;
  const uint32_t D_ = (uint32_t)d_inner;
  const uint32_t base = ((uint32_t)b * (uint32_t)seqlen + (uint32_t)min(t0, seqlen - 1)) * D_ + (uint32_t)(live ? d : 0);
  float a[kDiagWgLC], v[kDiagWgLC];
#pragma unroll
  for (int j = 0; j < kDiagWgLC; ++j) {
    const bool in = j < n;
    const uint32_t i = base + (uint32_t)(in ? j : 0) * D_;
    a[j] = in ? ld_at(dA, i) : 1.0f;
    v[j] = in ? ld_at(dBx, i) : 0.0f;
  }
  {
    float P = 1.0f, S = 0.0f;
#pragma unroll
    for (int j = 0; j < kDiagWgLC; ++j) {
      S = fmaf(a[j], S, v[j]);
      P *= a[j];
    }
    sP[k][c] = P;
    sS[k][c] = S;
  }
  __syncthreads();
  if (k == 0) {
    // the state entering each chunk, over its S
    float s = 0.0f;
    for (int kk = 0; kk < nck; ++kk) {
      const float P = sP[kk][c], S = sS[kk][c];
      sS[kk][c] = s;
      s = fmaf(P, s, S);
    }
  }
  __syncthreads();
  float s = sS[k][c];
  const float dd = live ? D[d] : 0.0f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    constexpr int kH = kDiagWgLC / 2;
    float cv[kH], xv[kH];
#pragma unroll
    for (int j = 0; j < kH; ++j) {
      const int jj = h * kH + j;
      const bool in = jj < n;
      const uint32_t i = base + (uint32_t)(in ? jj : 0) * D_;
      cv[j] = in ? ld_at(C, i) : 0.0f;
      xv[j] = in ? ld_at(x, i) : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kH; ++j) {
      const int jj = h * kH + j;
      s = fmaf(a[jj], s, v[jj]);
      if (jj < n) st_at(y, base + (uint32_t)jj * D_, fmaf(cv[j], s, dd * xv[j]));
    }
  }
}

// Backward of the diagonal recurrence (the gradient of the reference's
// sequential formula, kernels/hip/_torch_ops.py:346-386, and of its HIP
// kernel kernels/hip/selective_scan_backward.py:72-311), one lane per
// (batch, channel), channels coalesced. Pass 1 runs the recurrence forward
// and parks state[t] in grad_C; pass 2 runs backward in time:
//   grad_C[t]   = gy[t] * state[t]
//   g          += gy[t] * C[t]
//   grad_dA[t]  = g * state[t-1]
//   grad_dBx[t] = g
//   g          *= dA[t]
//   grad_x[t]   = gy[t] * D
// reading state[t] and state[t-1] from grad_C before step t overwrites
// entry t (entry t-1 is overwritten only at step t-1, later). Each lane also
// writes its sum over t of gy * x for the fixed-order batch reduction of
// grad_D. Loads run 8 steps ahead of the recurrence.
constexpr int kDiagU = 8;

__global__ void __launch_bounds__(256)
diag_scan_bwd_kernel(const float* __restrict__ dA, const float* __restrict__ dBx,
                     const float* __restrict__ C, const float* __restrict__ D,
                     const float* __restrict__ x, const float* __restrict__ gy,
                     float* __restrict__ g_dA, float* __restrict__ g_dBx, float* g_C,
                     float* __restrict__ g_x, float* __restrict__ gD_part, int batch, int seqlen,
                     int d_inner) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)batch * d_inner) return;
  const int b = (int)(gid / d_inner);
  const int d = (int)(gid % d_inner);
  const int64_t base = (int64_t)b * seqlen * d_inner + d;
  const int64_t D_ = d_inner;

  float s = 0.0f;
  int t = 0;
  for (; t + kDiagU <= seqlen; t += kDiagU) {
    float a[kDiagU], v[kDiagU];
#pragma unroll
    for (int k = 0; k < kDiagU; ++k) {
      a[k] = dA[base + (t + k) * D_];
      v[k] = dBx[base + (t + k) * D_];
    }
#pragma unroll
    for (int k = 0; k < kDiagU; ++k) {
      s = fmaf(a[k], s, v[k]);
      g_C[base + (t + k) * D_] = s;
    }
  }
  for (; t < seqlen; ++t) {
    s = fmaf(dA[base + t * D_], s, dBx[base + t * D_]);
    g_C[base + t * D_] = s;
  }

  const float dd = D[d];
  float g = 0.0f, gd = 0.0f;
  t = seqlen - 1;
  for (; t - kDiagU + 1 >= 0; t -= kDiagU) {
    float a[kDiagU], c[kDiagU], yv[kDiagU], xv[kDiagU], st[kDiagU + 1];
#pragma unroll
    for (int k = 0; k < kDiagU; ++k) {
      const int64_t i = base + (int64_t)(t - k) * D_;
      a[k] = dA[i];
      c[k] = C[i];
      yv[k] = gy[i];
      xv[k] = x[i];
      st[k] = g_C[i];
    }
    st[kDiagU] = t - kDiagU >= 0 ? g_C[base + (int64_t)(t - kDiagU) * D_] : 0.0f;
#pragma unroll
    for (int k = 0; k < kDiagU; ++k) {
      const int64_t i = base + (int64_t)(t - k) * D_;
      g_C[i] = yv[k] * st[k];
      g = fmaf(yv[k], c[k], g);
      g_dA[i] = g * st[k + 1];
      g_dBx[i] = g;
      g *= a[k];
      g_x[i] = yv[k] * dd;
      gd = fmaf(yv[k], xv[k], gd);
    }
  }
  for (; t >= 0; --t) {
    const int64_t i = base + (int64_t)t * D_;
    const float st_t = g_C[i];
    const float st_p = t > 0 ? g_C[i - D_] : 0.0f;
    const float yv = gy[i];
    g_C[i] = yv * st_t;
    g = fmaf(yv, C[i], g);
    g_dA[i] = g * st_p;
    g_dBx[i] = g;
    g *= dA[i];
    g_x[i] = yv * dd;
    gd = fmaf(yv, x[i], gd);
  }
  gD_part[gid] = gd;
}

// grad_D[d] = sum over b of gD_part[b][d], b in increasing order.
__global__ void __launch_bounds__(256)
diag_scan_gd_kernel(const float* __restrict__ gD_part, float* __restrict__ grad_D, int batch,
                    int d_inner) {
  const int d = blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= d_inner) return;
  float s = 0.0f;
  for (int b = 0; b < batch; ++b) s += gD_part[(int64_t)b * d_inner + d];
  grad_D[d] = s;
}

// The backward in chunks (lanes (batch, chunk, channel), the gradient
// buffers as scratch), for shapes whose (batch, channel) lanes are too few
// for the GPU. The adjoint is carried backward in time as c: g_t = gy_t C_t
// + c, then c = g_t dA_t is what step t passes to step t - 1, affine in c
// across a chunk. Four launches:
//   1. every chunk's aggregates in one pass over its rows: the forward decay
//      product and state from zero (P, S; every chunk but the last, in the
//      chunk's first two grad_C rows), the reverse product of dA and value of
//      c leaving the chunk from c = 0 (Q, G; every chunk but the first, in the
//      first rows of grad_dA and grad_x), and the chunk's sum of gy x (in the
//      first grad_dBx row);
//   2. per (batch, channel): the sums of gy x added in chunk order (into the
//      grad_D workspace), then the forward state entering each chunk (over
//      the sums) and the adjoint carried into each chunk,
//      c_k = Q_{k+1} c_{k+1} + G_{k+1} (over Q);
//   3. every chunk: its states from the state before it, then the
//      sequential kernel's backward sweep over them;
//   4. grad_D as the sum over the batch, in order.
// Every chunk but the last is full, so (P, S) fit its first two rows; each
// lane reads its chunk's scratch rows before it writes them. With kLC > 0
// (chunks of at most kLC steps) a lane holds its chunk's rows in registers:
// all its loads are issued together and the states never leave registers.
// With kLC = 0 the rows stream, and pass 3 parks the states in grad_C rows
// and reads them back from L2. Both do the same arithmetic in the same order
// (a register lane pads its steps past the chunk's end with dA = 1 and zeros,
// which leave every aggregate and sum unchanged).
template <int kLC>
__global__ void __launch_bounds__(256)
diag_bwd_aggs_kernel(const float* __restrict__ dA, const float* __restrict__ dBx,
                     const float* __restrict__ C, const float* __restrict__ gy,
                     const float* __restrict__ x, float* __restrict__ fwd_agg,
                     float* __restrict__ q_out, float* __restrict__ g_out,
                     float* __restrict__ gd_out, int batch, int seqlen, int d_inner, int lc,
                     int nchunks) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_b = (int64_t)nchunks * d_inner;
  if (gid >= (int64_t)batch * per_b) return;
  const int b = (int)(gid / per_b);
  const int k = (int)((gid % per_b) / d_inner);
  const int d = (int)(gid % d_inner);
  const int t0 = k * lc;
  const int n = min(lc, seqlen - t0);
  const int64_t D_ = d_inner;
  const int64_t first = ((int64_t)b * seqlen + t0) * D_ + d;
  float gd = 0.0f;
  if constexpr (kLC > 0) {
    // dA and dBx first (the forward aggregate), then C, gy and x (the reverse
    // one and the sum): at most about 64 loaded values live at once
    float a[kLC], v[kLC], cv[kLC], yv[kLC], xv[kLC];
#pragma unroll
    for (int j = 0; j < kLC; ++j) {
      const bool in = j < n;
      const int64_t i = first + (int64_t)(in ? j : 0) * D_;
      a[j] = in ? dA[i] : 1.0f;
      v[j] = in ? dBx[i] : 0.0f;
    }
    if (k + 1 < nchunks) {
      float P = 1.0f, S = 0.0f;
#pragma unroll
      for (int j = 0; j < kLC; ++j) {
        S = fmaf(a[j], S, v[j]);
        P *= a[j];
      }
      fwd_agg[first] = P;
      fwd_agg[first + D_] = S;
    }
#pragma unroll
    for (int j = 0; j < kLC; ++j) {
      const bool in = j < n;
      const int64_t i = first + (int64_t)(in ? j : 0) * D_;
      cv[j] = in ? C[i] : 0.0f;
      yv[j] = in ? gy[i] : 0.0f;
      xv[j] = in ? x[i] : 0.0f;
    }
    float c = 0.0f, Q = 1.0f;
#pragma unroll
    for (int j = kLC - 1; j >= 0; --j) {
      c = fmaf(yv[j], cv[j], c) * a[j];
      Q *= a[j];
      gd = fmaf(yv[j], xv[j], gd);
    }
    if (k > 0) {
      q_out[first] = Q;
      g_out[first] = c;
    }
  } else {
    if (k + 1 < nchunks) {
      int64_t idx = first;
      float P = 1.0f, S = 0.0f;
#pragma unroll 8
      for (int t = 0; t < n; ++t, idx += D_) {
        const float a = dA[idx];
        S = fmaf(a, S, dBx[idx]);
        P *= a;
      }
      fwd_agg[first] = P;
      fwd_agg[first + D_] = S;
    }
    int64_t idx = first + (int64_t)(n - 1) * D_;
    float c = 0.0f, Q = 1.0f;
#pragma unroll 8
    for (int t = n - 1; t >= 0; --t, idx -= D_) {
      const float a = dA[idx];
      const float yv = gy[idx];
      c = fmaf(yv, C[idx], c) * a;
      Q *= a;
      gd = fmaf(yv, x[idx], gd);
    }
    if (k > 0) {
      q_out[first] = Q;
      g_out[first] = c;
    }
  }
  gd_out[first] = gd;
}

// Per (batch, channel): the chunks' sums of gy x added in chunk order (into
// part), the forward state entering each chunk (over those sums, in
// grad_dBx's first rows) and the adjoint carried into each chunk from the
// right (over Q in grad_dA's first rows). Each round loads 16 chunks' worth
// of all three walks (the forward ones from the left, the reverse one from
// the right) before any of their rows is written, so the three dependent
// chains share their load latency; sx is read (sums) before it is written
// (states) through the one pointer.
__global__ void __launch_bounds__(256)
diag_bwd_carries_kernel(const float* __restrict__ fwd_agg, float* sx, float* __restrict__ q_c,
                        const float* __restrict__ g_agg, float* __restrict__ part, int batch,
                        int seqlen, int d_inner, int lc, int nchunks) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)batch * d_inner) return;
  const int b = (int)(gid / d_inner);
  const int d = (int)(gid % d_inner);
  constexpr int kG = 16;
  const int64_t base = (int64_t)b * seqlen * d_inner + d;
  const int64_t cs = (int64_t)lc * d_inner;
  float gd = 0.0f, s = 0.0f, c = 0.0f;
  for (int r0 = 0; r0 < nchunks; r0 += kG) {
    // forward walk: chunks r0 .. r0 + 15; reverse walk: chunks
    // nchunks - 1 - r0 down to nchunks - 16 - r0 (chunk 0 takes no Q / G)
    float G[kG], P[kG], S[kG], Q[kG], R[kG];
#pragma unroll
    for (int i = 0; i < kG; ++i) {
      const int kf = min(r0 + i, nchunks - 1);
      const int kp = min(r0 + i, max(nchunks - 2, 0));
      const int kr = max(nchunks - 1 - r0 - i, 1);
      G[i] = sx[base + kf * cs];
      P[i] = fwd_agg[base + kp * cs];
      S[i] = fwd_agg[base + kp * cs + d_inner];
      Q[i] = q_c[base + kr * cs];
      R[i] = g_agg[base + kr * cs];
    }
#pragma unroll
    for (int i = 0; i < kG; ++i) {
      const int kf = r0 + i;
      if (kf < nchunks) {
        gd += G[i];
        sx[base + kf * cs] = s;  // the state entering chunk kf
        if (kf + 1 < nchunks) s = fmaf(P[i], s, S[i]);
      }
      const int kr = nchunks - 1 - r0 - i;
      if (kr >= 1) {
        q_c[base + kr * cs] = c;  // the adjoint carried into chunk kr
        c = fmaf(Q[i], c, R[i]);
      }
    }
  }
  q_c[base] = c;
  part[gid] = gd;
}

// Both aggregates and all three carries of the chunked backward in one
// launch, for sequences of at most 1024 steps: the layout of
// diag_scan_wg_kernel (32 channels of one batch row per workgroup, one thread
// per (chunk of at most 32 steps, channel)). Per thread, the arithmetic of
// diag_bwd_aggs_kernel<32> in its order (dA and dBx first; then C, gy and x
// from the top half down, which continues the reverse walk and the gy x sum
// across the halves); then in LDS one thread per channel walks the forward
// states, one the adjoints and one the gy x sums, as diag_bwd_carries_kernel
// does. The entering state goes to the chunk's first grad_dBx row, the
// adjoint to its first grad_dA row and the channel's sum of gy x to the
// grad_D workspace: what diag_bwd_chunk_kernel<32> then reads.
__global__ void __launch_bounds__(1024)
diag_bwd_wg_carry_kernel(const float* __restrict__ dA, const float* __restrict__ dBx,
                         const float* __restrict__ C, const float* __restrict__ gy,
                         const float* __restrict__ x, float* __restrict__ s_in,
                         float* __restrict__ c_in, float* __restrict__ part, int batch,
                         int seqlen, int d_inner, int lc, int nck) {
  constexpr int kW = kDiagWgCh + 1;
  __shared__ float sP[kDiagWgLC][kW], sS[kDiagWgLC][kW], sQ[kDiagWgLC][kW], sG[kDiagWgLC][kW],
      sX[kDiagWgLC][kW];
  constexpr int kH = kDiagWgLC / 2;
  const int c = threadIdx.x % kDiagWgCh;
  const int k = threadIdx.x / kDiagWgCh;  // chunk (< nck <= 32)
  const int dblocks = (d_inner + kDiagWgCh - 1) / kDiagWgCh;
  const int b = blockIdx.x / dblocks;
  const int d = (blockIdx.x % dblocks) * kDiagWgCh + c;
  const bool live = d < d_inner;
  const int t0 = k * lc;
  const int n = live ? max(0, min(lc, seqlen - t0)) : 0;
  const uint32_t D_ = (uint32_t)d_inner;
  const uint32_t base = ((uint32_t)b * (uint32_t)seqlen + (uint32_t)min(t0, seqlen - 1)) * D_ + (uint32_t)(live ? d : 0);
  float a[kDiagWgLC];
  {
    float v[kDiagWgLC];
#pragma unroll
    for (int j = 0; j < kDiagWgLC; ++j) {
      const bool in = j < n;
      const uint32_t i = base + (uint32_t)(in ? j : 0) * D_;
      a[j] = in ? ld_at(dA, i) : 1.0f;
      v[j] = in ? ld_at(dBx, i) : 0.0f;
    }
    float P = 1.0f, S = 0.0f;
#pragma unroll
    for (int j = 0; j < kDiagWgLC; ++j) {
      S = fmaf(a[j], S, v[j]);
      P *= a[j];
    }
    sP[k][c] = P;
    sS[k][c] = S;
  }
  float cc = 0.0f, Q = 1.0f, gd = 0.0f;
  auto rev_half = [&](auto h_tag) {
    constexpr int h = decltype(h_tag)::value;
    float cv[kH], yv[kH], xv[kH];
#pragma unroll
    for (int j = 0; j < kH; ++j) {
      const int jj = h * kH + j;
      const bool in = jj < n;
      const uint32_t i = base + (uint32_t)(in ? jj : 0) * D_;
      cv[j] = in ? ld_at(C, i) : 0.0f;
      yv[j] = in ? ld_at(gy, i) : 0.0f;
      xv[j] = in ? ld_at(x, i) : 0.0f;
    }
#pragma unroll
    for (int j = kH - 1; j >= 0; --j) {
      cc = fmaf(yv[j], cv[j], cc) * a[h * kH + j];
      Q *= a[h * kH + j];
      gd = fmaf(yv[j], xv[j], gd);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  rev_half(std::integral_constant<int, 1>{});
  rev_half(std::integral_constant<int, 0>{});
  sQ[k][c] = Q;
  sG[k][c] = cc;
  sX[k][c] = gd;
  __syncthreads();
  const uint32_t first = base;  // the chunk's first row (chunks past the end have no rows)
  if (k == 0) {
    float s = 0.0f, g = 0.0f;
    for (int kk = 0; kk < nck; ++kk) {
      g += sX[kk][c];
      const float P = sP[kk][c], S = sS[kk][c];
      sS[kk][c] = s;  // the state entering chunk kk
      s = fmaf(P, s, S);
    }
    if (live) part[(int64_t)b * d_inner + d] = g;
  }
  if (k == (nck > 2 ? 2 : 0)) {
    float ca = 0.0f;
    for (int kk = nck - 1; kk >= 1; --kk) {
      const float Qk = sQ[kk][c], Gk = sG[kk][c];
      sG[kk][c] = ca;  // the adjoint entering chunk kk from the right
      ca = fmaf(Qk, ca, Gk);
    }
    sG[0][c] = ca;
  }
  __syncthreads();
  if (n > 0) {
    st_at(s_in, first, sS[k][c]);
    st_at(c_in, first, sG[k][c]);
  }
}

template <int kLC>
__global__ void __launch_bounds__(256)
diag_bwd_chunk_kernel(const float* __restrict__ dA, const float* __restrict__ dBx,
                      const float* __restrict__ C, const float* __restrict__ D,
                      const float* __restrict__ gy, float* __restrict__ g_dA,
                      float* __restrict__ g_dBx, float* g_C, float* __restrict__ g_x, int batch,
                      int seqlen, int d_inner, int lc, int nchunks) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_b = (int64_t)nchunks * d_inner;
  if (gid >= (int64_t)batch * per_b) return;
  const int b = (int)(gid / per_b);
  const int k = (int)((gid % per_b) / d_inner);
  const int d = (int)(gid % d_inner);
  const int t0 = k * lc;
  const int n = min(lc, seqlen - t0);
  const int64_t D_ = d_inner;
  const int64_t first = ((int64_t)b * seqlen + t0) * D_ + d;
  float c = g_dA[first];               // the adjoint carried into the chunk
  const float s_prev0 = g_dBx[first];  // the state before the chunk
  const float dd = D[d];
  auto step = [&](int t, float a, float cv, float yv, float st_t, float st_p) {
    const int64_t i = first + (int64_t)t * D_;
    g_C[i] = yv * st_t;
    const float g = fmaf(yv, cv, c);
    g_dA[i] = g * st_p;
    g_dBx[i] = g;
    c = g * a;
    g_x[i] = yv * dd;
  };
  if constexpr (kLC > 0) {
    float a[kLC], v[kLC], cv[kLC], yv[kLC], st[kLC + 1];
#pragma unroll
    for (int j = 0; j < kLC; ++j) {
      const bool in = j < n;
      const int64_t i = first + (int64_t)(in ? j : 0) * D_;
      a[j] = in ? dA[i] : 1.0f;
      v[j] = in ? dBx[i] : 0.0f;
      cv[j] = in ? C[i] : 0.0f;
      yv[j] = in ? gy[i] : 0.0f;
    }
    st[0] = s_prev0;
#pragma unroll
    for (int j = 0; j < kLC; ++j) st[j + 1] = fmaf(a[j], st[j], v[j]);
#pragma unroll
    for (int j = kLC - 1; j >= 0; --j)
      if (j < n) step(j, a[j], cv[j], yv[j], st[j + 1], st[j]);
  } else {
    {
      // the chunk's states, from the state before it, into its grad_C rows
      // (read back below from L2 by this lane)
      float sv = s_prev0;
      int64_t j = first;
#pragma unroll 8
      for (int t = 0; t < n; ++t, j += D_) {
        sv = fmaf(dA[j], sv, dBx[j]);
        g_C[j] = sv;
      }
    }
    // steps t .. t - 7 (chunk-relative) loaded before any of their rows is
    // written: grad_C holds the states and is overwritten with gy * state, so
    // the loads cannot move past the stores otherwise
    int t = n - 1;
    for (; t - kDiagU + 1 >= 0; t -= kDiagU) {
      float a[kDiagU], cv[kDiagU], yv[kDiagU], st[kDiagU + 1];
#pragma unroll
      for (int j = 0; j < kDiagU; ++j) {
        const int64_t i = first + (int64_t)(t - j) * D_;
        a[j] = dA[i];
        cv[j] = C[i];
        yv[j] = gy[i];
        st[j] = g_C[i];
      }
      st[kDiagU] = t - kDiagU >= 0 ? g_C[first + (int64_t)(t - kDiagU) * D_] : s_prev0;
#pragma unroll
      for (int j = 0; j < kDiagU; ++j) step(t - j, a[j], cv[j], yv[j], st[j], st[j + 1]);
    }
    for (; t >= 0; --t) {
      const int64_t i = first + (int64_t)t * D_;
      const float st_t = g_C[i];
      const float st_p = t > 0 ? g_C[i - D_] : s_prev0;
      step(t, dA[i], C[i], gy[i], st_t, st_p);
    }
  }
}

// ---------------------------------------------------------------------------
// Mamba-1 backward (the gradient of selective_scan_ref; the reference's
// kernel is external/mamba/csrc/selective_scan/selective_scan_bwd_kernel.cuh,
// entry point selective_scan.cpp:339-490). With delta' = softplus?(delta +
// bias), a_l = exp(delta'_l A_n), dy_l = dout_l * silu(z_l), and g_l the
// gradient of the state h_l:
//   g_l        = a_{l+1} g_{l+1} + dy_l C_l
//   dB[n, l]  += g_l delta'_l u_l                    (summed over channels)
//   dC[n, l]  += dy_l h_l                            (summed over channels)
//   du_l       = D dy_l + sum_n g_l delta'_l B_l
//   ddelta'_l  = sum_n g_l (u_l B_l + A_n a_l h_{l-1})
//   dA[n]     += g_l delta'_l a_l h_{l-1}
//   dD        += dy_l u_l,  dz_l = dout_l y_l silu'(z_l)
//   ddelta_l   = ddelta'_l * sigmoid(delta_l + bias) with softplus below its
//                threshold 20, else ddelta'_l;  dbias += ddelta_l
// Three launches. The preparation pass (mamba_scan_fwd_kernel<..., true>)
// runs the recurrence forward, saves the state before every 16-step block
// and writes dz. The reverse pass (mamba_scan_bwd_kernel) walks the 64-step
// tiles from last to first with the forward's lane decomposition (lane =
// channel c x state n): per 16-step block it recomputes a_l and h_l from the
// saved state, then runs g backwards. Sums over states (du, ddelta) go
// through a per-wave LDS transpose as in the forward; sums over the four
// channels of a wave (dB, dC) through two permlane swaps that also
// distribute the results over the lanes, then over the four waves through
// LDS, and over channel tiles in the final pass (scan_bwd_finalize_kernel)
// in a fixed order, so every gradient is deterministic.
// ---------------------------------------------------------------------------
template <typename TU, typename TD, typename TBC, bool kSoftplus>
__global__ void __launch_bounds__(256)
mamba_scan_bwd_kernel(ScanParams p) {
  __shared__ float Bs[16 * kBStride];                  // B[n][t] of the tile
  __shared__ float Cs[16 * kBStride];                  // C[n][t] of the tile
  __shared__ __align__(16) float tbuf[4][4 * kTC];     // per wave: (g B, A w)[c][j][n]
  __shared__ float wbuf[4][64 * kWP];                  // per wave: (dB, dC) channel sums [lane][pair]

  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int c = lane / 16;
  const int n = lane % 16;

  const int per_batch = p.ngroups * p.tiles_per_group;
  const int b = blockIdx.x / per_batch;
  const int g = (blockIdx.x % per_batch) / p.tiles_per_group;
  const int tile = blockIdx.x % p.tiles_per_group;
  const int ch_local = tile * kScanCh + wave * 4 + c;
  const bool ch_ok = ch_local < p.ch_per_group;
  const int d = g * p.ch_per_group + (ch_ok ? ch_local : 0);
  const bool n_ok = n < p.dstate;
  const int n_c = min(n, p.dstate - 1);

  const float a_nat = (ch_ok && n_ok) ? p.A[(int64_t)d * p.A_ds + n] : 0.0f;
  const float a_scaled = a_nat * kLog2e;
  const float dbias = p.delta_bias ? p.delta_bias[d] : 0.0f;
  const float dskip = p.D ? p.D[d] : 0.0f;

  const int64_t u_row = (int64_t)b * p.u_bs + (int64_t)d * p.u_ds;
  const int64_t d_row = (int64_t)b * p.d_bs + (int64_t)d * p.d_ds;
  const int64_t z_row = (int64_t)b * p.z_bs + (int64_t)d * p.z_ds;
  const int64_t o_row = (int64_t)b * p.o_bs + (int64_t)d * p.o_ds;
  const int64_t go_row = (int64_t)b * p.go_bs + (int64_t)d * p.go_ds;
  const int64_t B_base = (int64_t)b * p.B_bs + (int64_t)g * p.B_gs;
  const int64_t C_base = (int64_t)b * p.C_bs + (int64_t)g * p.C_gs;
  const int sn = tid / 16, q = tid % 16;
  const int sn_c = min(sn, p.dstate - 1);
  const int last_l = p.seqlen - 1;

  float* tb = tbuf[wave];
  float* wb = wbuf[wave];

  // Global loads of one 64-step tile, issued a tile ahead of their use
  // (clamped, always-valid addresses; masking and conversion at the use).
  struct TileRegs {
    TBC bv[4], cv[4];                    // staging: state sn, steps 4q .. 4q + 3
    TD dv[4];                            // broadcast sources: steps 4n .. 4n + 3
    TU uv[4], gv[4], zv[4];
    TD dr[4];                            // reducer role: steps 16 blk + n
    TU ur[4], gr[4], zr[4], yr[4];       // yr: the forward's pre-gate output (saved-states path)
    float ck[4];                         // states before the tile's four blocks
  };
  const TU* const zsrc = static_cast<const TU*>(p.z ? p.z : p.u);  // without z: unused u loads
  const int64_t zrow = p.z ? z_row : u_row;
  // the forward's pre-gate output (contiguous, as du), given on the saved-states path
  const TU* const ysrc = static_cast<const TU*>(p.out_prez ? p.out_prez : p.u);
  const int64_t yrow = p.out_prez ? o_row : u_row;
  const int64_t ck_row = (int64_t)d * p.dstate + n_c;
  auto load_tile = [&](int l0, TileRegs& r) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int lc = min(l0 + 4 * q + k, last_l);
      r.bv[k] = static_cast<const TBC*>(p.B)[B_base + (int64_t)sn_c * p.B_ns + lc];
      r.cv[k] = static_cast<const TBC*>(p.C)[C_base + (int64_t)sn_c * p.C_ns + lc];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int lc = min(l0 + 4 * n + k, last_l);
      r.dv[k] = static_cast<const TD*>(p.delta)[d_row + lc];
      r.uv[k] = static_cast<const TU*>(p.u)[u_row + lc];
      r.gv[k] = static_cast<const TU*>(p.dout)[go_row + lc];
      r.zv[k] = zsrc[zrow + lc];
    }
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int lc = min(l0 + 16 * blk + n, last_l);
      r.dr[blk] = static_cast<const TD*>(p.delta)[d_row + lc];
      r.ur[blk] = static_cast<const TU*>(p.u)[u_row + lc];
      r.gr[blk] = static_cast<const TU*>(p.dout)[go_row + lc];
      r.zr[blk] = zsrc[zrow + lc];
      r.yr[blk] = ysrc[yrow + lc];
      const int chunk = min((l0 + 16 * blk) / kCk, p.nchunks - 1);
      r.ck[blk] = p.ck[((int64_t)b * p.nchunks + chunk) * p.dim * p.dstate + ck_row];
    }
  };
  // dy = dout * silu(z) (dout without a gate)
  auto gated = [&](float go, float zv) { return p.z ? go * zv * sigmoid_f32(zv) : go; };

  float gs = 0.0f;       // gradient of the state after the step being processed
  float a_next = 0.0f;   // decay of the step after it
  float dA_acc = 0.0f;
  float dD_acc = 0.0f, dbias_acc = 0.0f;  // reducer role: channel c, steps 16 blk + n

  TileRegs cur, nxt{};
  load_tile((last_l / kScanT) * kScanT, cur);
  for (int l0 = (last_l / kScanT) * kScanT; l0 >= 0; l0 -= kScanT) {
    __syncthreads();  // the previous tile's readers of Bs / Cs / wbuf are done
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const bool ok = sn < p.dstate && l0 + 4 * q + k < p.seqlen;
      Bs[sn * kBStride + 4 * q + k] = ok ? to_f32(cur.bv[k]) : 0.0f;
      Cs[sn * kBStride + 4 * q + k] = ok ? to_f32(cur.cv[k]) : 0.0f;
    }
    // broadcast sources: steps 4n .. 4n + 3 of channel c
    float bd[4], bdu[4], bdy[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const bool ok = ch_ok && l0 + 4 * n + k < p.seqlen;
      float dv = to_f32(cur.dv[k]) + dbias;
      if constexpr (kSoftplus) dv = softplus_f32(dv);
      bd[k] = ok ? dv : 0.0f;
      bdu[k] = bd[k] * to_f32(cur.uv[k]);
      bdy[k] = ok ? gated(to_f32(cur.gv[k]), to_f32(cur.zv[k])) : 0.0f;
    }
    asm volatile("s_nop 1"
                 : "+v"(bd[0]), "+v"(bd[1]), "+v"(bd[2]), "+v"(bd[3]), "+v"(bdu[0]), "+v"(bdu[1]),
                   "+v"(bdu[2]), "+v"(bdu[3]), "+v"(bdy[0]), "+v"(bdy[1]), "+v"(bdy[2]), "+v"(bdy[3]));
    if (l0 > 0) load_tile(l0 - kScanT, nxt);
    // keep the compiler from sinking the prefetch towards its use
    asm volatile("" ::: "memory");
    __syncthreads();

    auto block = [&](auto blk_c) {
      constexpr int BLK = decltype(blk_c)::value;
      const int lb = l0 + 16 * BLK;
      if (lb >= p.seqlen) return;  // workgroup-uniform
      const float hstart = (ch_ok && n_ok) ? cur.ck[BLK] : 0.0f;
      float bt[16], ct[16], as[16], hs[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        bt[j] = Bs[n * kBStride + 16 * BLK + j];
        ct[j] = Cs[n * kBStride + 16 * BLK + j];
      }
      // recompute the block's decays and states
      float xv[16];
      static_for<0, 16>([&](auto j_c) {
        constexpr int J = decltype(j_c)::value;
        constexpr int kSrc = 4 * BLK + J / 4;
        as[J] = mul_bcast<kSrc>(bd[J % 4], a_scaled);
        xv[J] = mul_bcast<kSrc>(bdu[J % 4], bt[J]);
      });
#pragma unroll
      for (int j = 0; j < 16; ++j) as[j] = __builtin_amdgcn_exp2f(as[j]);
      float h = hstart;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        h = fmaf(as[j], h, xv[j]);
        hs[j] = h;
      }
      // reverse over the block; (dB, dC) contributions of steps 2i, 2i + 1
      // are folded over channels as soon as both exist
      float pB = 0.0f, pC = 0.0f;
      static_for<0, 16>([&](auto i_c) {
        constexpr int J = 15 - decltype(i_c)::value;
        constexpr int kSrc = 4 * BLK + J / 4;
        constexpr int K = J % 4;
        gs = fmaf(gs, a_next, mul_bcast<kSrc>(bdy[K], ct[J]));
        a_next = as[J];
        const float hp = J > 0 ? hs[J > 0 ? J - 1 : 0] : hstart;
        // w = g a h_{l-1}: dA += delta' w; the state sums of g B and A w
        // give du = delta' sum(g B) + D dy and ddelta' = u sum(g B) + sum(A w)
        // (delta' and u are common to the 16 states of a step)
        const float w = gs * (as[J] * hp);
        const float gB = gs * bt[J];
        dA_acc = fma_bcast<kSrc>(bd[K], w, dA_acc);
        const float cB = mul_bcast<kSrc>(bdu[K], gs);
        const float cC = mul_bcast<kSrc>(bdy[K], hs[J]);
        *reinterpret_cast<float2*>(&tb[c * kTC + J * kTJ + 2 * n]) = make_float2(gB, a_nat * w);
        if constexpr (J % 2 == 1) {
          pB = cB;
          pC = cC;
        } else {
          // lanes 16 r + n: r = 0: dB at step J, 1: dB at J + 1, 2: dC at J, 3: dC at J + 1
          const float s_even = swap32_sum(cB, cC);
          const float s_odd = swap32_sum(pB, pC);
          wb[lane * kWP + 8 * BLK + J / 2] = swap16_sum(s_even, s_odd);
        }
      });
      __builtin_amdgcn_wave_barrier();
      // lane (c, j = n): sums over the 16 states of step lb + n
      float sgb = 0.0f, saw = 0.0f;
#pragma unroll
      for (int s4 = 0; s4 < 8; ++s4) {
        const float4 v = *reinterpret_cast<const float4*>(&tb[c * kTC + n * kTJ + 4 * s4]);
        sgb += v.x + v.z;
        saw += v.y + v.w;
      }
      __builtin_amdgcn_wave_barrier();
      const int l = lb + n;
      if (ch_ok && l < p.seqlen) {
        const float go = to_f32(cur.gr[BLK]);
        float dyv = go;  // dout * silu(z), or dout without a gate
        if (p.z) {
          const float zv = to_f32(cur.zr[BLK]);
          const float sg = sigmoid_f32(zv);
          dyv = go * zv * sg;
          // saved-states path: dz = dout * y * s * (1 + z (1 - s)) from the
          // forward's pre-gate output y, s = sigmoid(z)
          if (p.out_prez)
            static_cast<TU*>(p.dz)[o_row + l] =
                from_f32<TU>(go * to_f32(cur.yr[BLK]) * sg * fmaf(zv, 1.0f - sg, 1.0f));
        }
        const float uv = to_f32(cur.ur[BLK]);
        const float x = to_f32(cur.dr[BLK]) + dbias;
        float dlt = x, ddl = fmaf(uv, sgb, saw);
        if constexpr (kSoftplus) {
          dlt = softplus_f32(x);
          if (x <= 20.0f) ddl *= sigmoid_f32(x);
        }
        static_cast<TU*>(p.du)[o_row + l] = from_f32<TU>(fmaf(dskip, dyv, dlt * sgb));
        static_cast<TD*>(p.ddelta)[o_row + l] = from_f32<TD>(ddl);
        dD_acc = fmaf(dyv, uv, dD_acc);
        dbias_acc += ddl;
      }
    };
    block(std::integral_constant<int, 3>{});
    block(std::integral_constant<int, 2>{});
    block(std::integral_constant<int, 1>{});
    block(std::integral_constant<int, 0>{});

    __syncthreads();  // wbuf holds the tile's per-wave sums
    {
      const int t = tid % 64, ng = tid / 64;
      const int l = l0 + t;
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        float* part = v ? p.dC_part : p.dB_part;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n2 = 4 * ng + i;
          const int L = 16 * (2 * v + (t & 1)) + n2;
          const float sum = ((wbuf[0][L * kWP + t / 2] + wbuf[1][L * kWP + t / 2]) +
                             wbuf[2][L * kWP + t / 2]) + wbuf[3][L * kWP + t / 2];
          if (n2 < p.dstate && l < p.seqlen)
            part[((((int64_t)tile * p.batch + b) * p.ngroups + g) * p.dstate + n2) * p.seqlen + l] = sum;
        }
      }
    }
    cur = nxt;
  }
  if (ch_ok && n_ok) p.dA_part[((int64_t)b * p.dim + d) * p.dstate + n] = dA_acc;
  dD_acc = row16_sum(dD_acc);
  dbias_acc = row16_sum(dbias_acc);
  if (ch_ok && n == 0) {
    p.dD_part[(int64_t)b * p.dim + d] = dD_acc;
    p.dbias_part[(int64_t)b * p.dim + d] = dbias_acc;
  }
}

// Arguments of the final sums (scan_bwd_finalize_kernel, and the tail blocks
// of scan_bwd_bc_sum4_kernel).
template <typename TBC>
struct FinArgs {
  const float *dB_part, *dC_part, *dA_part, *dBc_part, *dCc_part, *dD_part, *dbias_part;
  TBC *dB, *dC;
  float *dA, *dBc, *dCc, *dD, *dbias;
  int64_t nbc;  // dB / dC elements summed here (0 when the vector pass did them)
  int tiles, nb, dim, dstate;
};

// Items i0, i0 + stride, ... of the final sums: dB / dC over channel tiles
// (the first 2 nbc items), then dA / dB / dC of input-independent B / C and
// dD / ddelta_bias over the batch, each in increasing order.
template <typename TBC>
__device__ void finalize_items(const FinArgs<TBC>& a, int64_t i0, int64_t stride) {
  const int64_t nA = (int64_t)a.dim * a.dstate;
  const int64_t total = 2 * a.nbc + 3 * nA + 2 * (int64_t)a.dim;
  for (int64_t i = i0; i < total; i += stride) {
    if (i < 2 * a.nbc) {
      const bool is_c = i >= a.nbc;
      const int64_t e = is_c ? i - a.nbc : i;
      TBC* dst = is_c ? a.dC : a.dB;
      if (!dst) continue;
      const float* part = is_c ? a.dC_part : a.dB_part;
      float s = 0.0f;
      for (int t = 0; t < a.tiles; ++t) s += part[(int64_t)t * a.nbc + e];
      dst[e] = from_f32<TBC>(s);
      continue;
    }
    int64_t e = i - 2 * a.nbc;
    if (e < 3 * nA) {
      const int k = (int)(e / nA);
      e -= k * nA;
      float* dst = k == 0 ? a.dA : k == 1 ? a.dBc : a.dCc;
      if (!dst) continue;
      const float* part = k == 0 ? a.dA_part : k == 1 ? a.dBc_part : a.dCc_part;
      float s = 0.0f;
      for (int bb = 0; bb < a.nb; ++bb) s += part[(int64_t)bb * nA + e];
      dst[e] = s;
      continue;
    }
    e -= 3 * nA;
    const bool is_bias = e >= a.dim;
    const int dd = (int)(is_bias ? e - a.dim : e);
    float* dst = is_bias ? a.dbias : a.dD;
    if (!dst) continue;
    const float* part = is_bias ? a.dbias_part : a.dD_part;
    float s = 0.0f;
    for (int bb = 0; bb < a.nb; ++bb) s += part[(int64_t)bb * a.dim + dd];
    dst[dd] = s;
  }
}

// dB / dC = sum over channel tiles of the partial rows, 4 elements per
// thread (16-byte loads, up to 16 tiles in flight), tiles in increasing
// order: the same order, hence the same bits, as scan_bwd_finalize_kernel.
// Blocks from sum_blocks on run the remaining final sums (fa, with nbc = 0)
// in the same launch.
template <typename TBC>
__global__ void __launch_bounds__(256)
scan_bwd_bc_sum4_kernel(const float* __restrict__ dB_part, const float* __restrict__ dC_part,
                        TBC* __restrict__ dB, TBC* __restrict__ dC, int64_t n4, int tiles,
                        unsigned sum_blocks, FinArgs<TBC> fa) {
  struct alignas(4 * sizeof(TBC)) Out4 {
    TBC v[4];
  };
  if (blockIdx.x >= sum_blocks) {
    finalize_items(fa, (int64_t)(blockIdx.x - sum_blocks) * blockDim.x + threadIdx.x,
                   (int64_t)(gridDim.x - sum_blocks) * blockDim.x);
    return;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < 2 * n4;
       i += (int64_t)sum_blocks * blockDim.x) {
    const bool is_c = i >= n4;
    const int64_t e4 = is_c ? i - n4 : i;
    if (!(is_c ? dC : dB)) continue;
    const float4* part = reinterpret_cast<const float4*>(is_c ? dC_part : dB_part) + e4;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    int t = 0;
    // 16 loads in flight per lane: at 2 waves per SIMD (the C5 shape) the
    // latency of each round is exposed, so fewer, wider rounds
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4* pv = reinterpret_cast<const f32x4*>(part);
    for (; t + 16 <= tiles; t += 16) {
      f32x4 v[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) v[k] = __builtin_nontemporal_load(pv + (int64_t)(t + k) * n4);
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        acc.x += v[k][0];
        acc.y += v[k][1];
        acc.z += v[k][2];
        acc.w += v[k][3];
      }
    }
    for (; t + 8 <= tiles; t += 8) {
      float4 v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = part[(int64_t)(t + k) * n4];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        acc.x += v[k].x;
        acc.y += v[k].y;
        acc.z += v[k].z;
        acc.w += v[k].w;
      }
    }
    for (; t < tiles; ++t) {
      const float4 v = part[(int64_t)t * n4];
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    Out4 o;
    o.v[0] = from_f32<TBC>(acc.x);
    o.v[1] = from_f32<TBC>(acc.y);
    o.v[2] = from_f32<TBC>(acc.z);
    o.v[3] = from_f32<TBC>(acc.w);
    reinterpret_cast<Out4*>(is_c ? dC : dB)[e4] = o;
  }
}

// Fixed-order sums of the reverse pass's partial results:
//   dB / dC [b, g, n, l] = sum over the channel tiles of the group (variable B / C)
//   dA [d, n], constant dB / dC [d, n], dD [d], dbias [d] = sum over the batch
// A null destination is skipped; nb = 0 (no steps) writes zeros.
template <typename TBC>
__global__ void __launch_bounds__(256) scan_bwd_finalize_kernel(FinArgs<TBC> a) {
  finalize_items(a, (int64_t)blockIdx.x * blockDim.x + threadIdx.x, (int64_t)gridDim.x * blockDim.x);
}

// Whether the fast kernel's layout assumptions hold: whole 64-step tiles,
// whole 16-channel workgroups, 4-element aligned rows for the vector loads,
// and every buffer resource's extent (16 channel rows, or dstate B / C rows)
// below 2 GiB.
template <typename TU, typename TD, typename TBC>
bool scan_fast_ok(const ScanParams& p, bool prep = false, int wgc = kScanCh) {
  auto al4 = [](const void* ptr, int64_t s0, int64_t s1, int64_t s2, size_t esz) {
    return (reinterpret_cast<uintptr_t>(ptr) % (4 * esz)) == 0 && s0 % 4 == 0 && s1 % 4 == 0 &&
           s2 % 4 == 0;
  };
  auto fits = [&](int64_t rows, int64_t pitch, size_t esz) {
    return pitch >= 0 && ((rows - 1) * pitch + p.seqlen) * (int64_t)esz < ((int64_t)1 << 31);
  };
  if (p.seqlen % kScanT != 0 || p.ch_per_group % wgc != 0) return false;
  if (!al4(p.u, p.u_bs, p.u_ds, 0, sizeof(TU)) || !al4(p.delta, p.d_bs, p.d_ds, 0, sizeof(TD)))
    return false;
  if (!al4(p.B, p.B_bs, p.B_gs, p.B_ns, sizeof(TBC)) || !al4(p.C, p.C_bs, p.C_gs, p.C_ns, sizeof(TBC)))
    return false;
  if (p.u_bs < 0 || p.d_bs < 0 || p.o_bs < 0 || p.z_bs < 0 || p.B_bs < 0 || p.C_bs < 0 ||
      p.B_gs < 0 || p.C_gs < 0)
    return false;
  if (prep && (p.go_bs < 0 || !fits(wgc, p.go_ds, sizeof(TU)))) return false;
  if (p.ck && (int64_t)p.nchunks * p.dim * p.dstate * 4 >= ((int64_t)1 << 31)) return false;
  return fits(wgc, p.u_ds, sizeof(TU)) && fits(wgc, p.d_ds, sizeof(TD)) &&
         fits(wgc, p.o_ds, sizeof(TU)) && (!p.z || fits(wgc, p.z_ds, sizeof(TU))) &&
         fits(p.dstate, p.B_ns, sizeof(TBC)) && fits(p.dstate, p.C_ns, sizeof(TBC));
}

template <typename TU, typename TD, typename TBC>
void launch_scan(const ScanParams& p, hipStream_t s) {
  const int grid = p.batch * p.ngroups * p.tiles_per_group;
  const bool lean = p.z && !p.out_prez && !p.ck && !p.chunk_states;
  const bool train = p.z && p.out_prez && p.ck && !p.chunk_states;
  // whole tiles: producer / consumer waves (inference and training variants
  // fixed at compile time, any other combination of outputs at run time)
  if (scan_fast_ok<TU, TD, TBC>(p) && lean && p.softplus)
    mamba_scan_split_kernel<TU, TD, TBC, true, kFwdLean><<<dim3(grid), dim3(512), 0, s>>>(p);
  else if (scan_fast_ok<TU, TD, TBC>(p) && lean)
    mamba_scan_split_kernel<TU, TD, TBC, false, kFwdLean><<<dim3(grid), dim3(512), 0, s>>>(p);
  else if (scan_fast_ok<TU, TD, TBC>(p) && train && p.softplus)
    mamba_scan_split_kernel<TU, TD, TBC, true, kFwdTrain><<<dim3(grid), dim3(512), 0, s>>>(p);
  else if (scan_fast_ok<TU, TD, TBC>(p) && train)
    mamba_scan_split_kernel<TU, TD, TBC, false, kFwdTrain><<<dim3(grid), dim3(512), 0, s>>>(p);
  else if (scan_fast_ok<TU, TD, TBC>(p) && p.softplus)
    mamba_scan_split_kernel<TU, TD, TBC, true, kFwdAny><<<dim3(grid), dim3(512), 0, s>>>(p);
  else if (scan_fast_ok<TU, TD, TBC>(p))
    mamba_scan_split_kernel<TU, TD, TBC, false, kFwdAny><<<dim3(grid), dim3(512), 0, s>>>(p);
  else
    mamba_scan_fwd_kernel<TU, TD, TBC><<<dim3(grid), dim3(256), 0, s>>>(p);
}

// dstate in (16, 64] with variable B / C: the specialised kernel with 2 or 4
// rows per channel, when the whole-tile conditions hold. Returns whether it
// launched.
template <typename TU, typename TD, typename TBC>
bool launch_scan_rows(const ScanParams& p, hipStream_t s) {
  const int rpc = p.dstate <= 32 ? 2 : 4;
  const int wgc = kScanCh / rpc;
  if (p.dstate <= 16 || p.dstate > 64 || p.b_const || p.c_const) return false;
  if (!scan_fast_ok<TU, TD, TBC>(p, false, wgc)) return false;
  ScanParams q = p;
  q.tiles_per_group = p.ch_per_group / wgc;
  const int grid = q.batch * q.ngroups * q.tiles_per_group;
  if (rpc == 2) {
    if (p.softplus) mamba_scan_fast_kernel<TU, TD, TBC, true, false, 2><<<dim3(grid), dim3(256), 0, s>>>(q);
    else mamba_scan_fast_kernel<TU, TD, TBC, false, false, 2><<<dim3(grid), dim3(256), 0, s>>>(q);
  } else {
    if (p.softplus) mamba_scan_fast_kernel<TU, TD, TBC, true, false, 4><<<dim3(grid), dim3(256), 0, s>>>(q);
    else mamba_scan_fast_kernel<TU, TD, TBC, false, false, 4><<<dim3(grid), dim3(256), 0, s>>>(q);
  }
  return true;
}

template <typename TU>
bool dispatch_scan_rows(const ScanParams& p, int u_dtype, int delta_dtype, int bc_dtype, hipStream_t s) {
  const bool d32 = delta_dtype == AK_DTYPE_F32;
  const bool bc32 = bc_dtype == AK_DTYPE_F32;
  if (!d32 && delta_dtype != u_dtype) return false;
  if (!bc32 && bc_dtype != u_dtype) return false;
  if (d32 && bc32) return launch_scan_rows<TU, float, float>(p, s);
  if (d32) return launch_scan_rows<TU, float, TU>(p, s);
  if (bc32) return launch_scan_rows<TU, TU, float>(p, s);
  return launch_scan_rows<TU, TU, TU>(p, s);
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

// The backward's finish pass: fixed-order sums of the reverse pass's
// partials into the gradients. A variable dB / dC comes out in TBC, a
// constant one ([dim, dstate]) in fp32.
template <typename TBC>
void scan_bwd_finish(const ScanParams& p, void* dB, void* dC, float* dA, float* dD, float* dbias,
                     hipStream_t s) {
  TBC* dBv = p.b_const ? nullptr : static_cast<TBC*>(dB);
  TBC* dCv = p.c_const ? nullptr : static_cast<TBC*>(dC);
  float* dBk = p.b_const ? static_cast<float*>(dB) : nullptr;
  float* dCk = p.c_const ? static_cast<float*>(dC) : nullptr;
  int64_t nbc = (dBv || dCv) ? (int64_t)p.batch * p.ngroups * p.dstate * p.seqlen : 0;
  const size_t out4 = 4 * sizeof(TBC);
  auto al4 = [&](const void* q) { return !q || reinterpret_cast<uintptr_t>(q) % out4 == 0; };
  FinArgs<TBC> fa{p.dB_part, p.dC_part, p.dA_part, p.dBc_part, p.dCc_part, p.dD_part, p.dbias_part,
                  dBv, dCv, dA, dBk, dCk, dD, dbias, nbc, p.tiles_per_group, p.batch, p.dim, p.dstate};
  if (nbc > 0 && nbc % 4 == 0 && al4(dBv) && al4(dCv)) {
    // one launch: the vector dB / dC sums, then blocks for the per-batch sums
    const int64_t n4 = nbc / 4;
    const unsigned blocks4 = (unsigned)std::min<int64_t>((2 * n4 + 255) / 256, 65535);
    fa.nbc = 0;
    const int64_t rest = 3 * (int64_t)p.dim * p.dstate + 2 * (int64_t)p.dim;
    const unsigned fin_blocks = (unsigned)std::min<int64_t>((rest + 255) / 256, 8192);
    scan_bwd_bc_sum4_kernel<TBC><<<dim3(blocks4 + fin_blocks), dim3(256), 0, s>>>(
        p.dB_part, p.dC_part, dBv, dCv, n4, p.tiles_per_group, blocks4, fa);
    return;
  }
  const int64_t total = 2 * nbc + 3 * (int64_t)p.dim * p.dstate + 2 * (int64_t)p.dim;
  const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 8192);
  scan_bwd_finalize_kernel<TBC><<<dim3(blocks), dim3(256), 0, s>>>(fa);
}

int finish_for(int bc_dtype, const ScanParams& p, void* dB, void* dC, float* dA, float* dD,
               float* dbias, hipStream_t s) {
  switch (bc_dtype) {
    case AK_DTYPE_F32: scan_bwd_finish<float>(p, dB, dC, dA, dD, dbias, s); break;
    case AK_DTYPE_F16: scan_bwd_finish<f16>(p, dB, dC, dA, dD, dbias, s); break;
    default: scan_bwd_finish<bf16>(p, dB, dC, dA, dD, dbias, s); break;
  }
  return 0;
}

template <typename T>
constexpr int dtype_code_of() {
  return std::is_same_v<T, float> ? AK_DTYPE_F32 : (std::is_same_v<T, f16> ? AK_DTYPE_F16 : AK_DTYPE_BF16);
}

// With the forward's states (p.ck) and pre-gate output (p.out_prez) saved,
// the preparation pass is skipped: the reverse pass restarts from the saved
// states and computes dz itself.
template <typename TU, typename TD, typename TBC>
void launch_scan_bwd(const ScanParams& p, void* dB, void* dC, float* dA, float* dD, float* dbias,
                     bool saved_states, hipStream_t s) {
  const int grid = p.batch * p.ngroups * p.tiles_per_group;
  if (!saved_states) {  // preparation pass: states every 16 steps and dz
    if (scan_fast_ok<TU, TD, TBC>(p, true) && p.z && p.softplus)
      mamba_scan_split_kernel<TU, TD, TBC, true, kPrepGated><<<dim3(grid), dim3(512), 0, s>>>(p);
    else if (scan_fast_ok<TU, TD, TBC>(p, true) && p.z)
      mamba_scan_split_kernel<TU, TD, TBC, false, kPrepGated><<<dim3(grid), dim3(512), 0, s>>>(p);
    else if (scan_fast_ok<TU, TD, TBC>(p, true) && p.softplus)
      mamba_scan_fast_kernel<TU, TD, TBC, true, true><<<dim3(grid), dim3(256), 0, s>>>(p);
    else if (scan_fast_ok<TU, TD, TBC>(p, true))
      mamba_scan_fast_kernel<TU, TD, TBC, false, true><<<dim3(grid), dim3(256), 0, s>>>(p);
    else
      mamba_scan_fwd_kernel<TU, TD, TBC, true><<<dim3(grid), dim3(256), 0, s>>>(p);
  }
  ScanParams q = p;  // the whole-tile pass may write fewer, wider dB / dC partial rows
  if (launch_scan_bwd_fast(q, dtype_code_of<TU>(), dtype_code_of<TD>(), dtype_code_of<TBC>(), s)) {
    // whole tiles: the buffer-resource reverse pass
  } else if (p.softplus) {
    mamba_scan_bwd_kernel<TU, TD, TBC, true><<<dim3(grid), dim3(256), 0, s>>>(p);
  } else {
    mamba_scan_bwd_kernel<TU, TD, TBC, false><<<dim3(grid), dim3(256), 0, s>>>(p);
  }
  scan_bwd_finish<TBC>(q, dB, dC, dA, dD, dbias, s);
}

template <typename TU>
int dispatch_scan_bwd(const ScanParams& p, int u_dtype, int delta_dtype, int bc_dtype, void* dB,
                      void* dC, float* dA, float* dD, float* dbias, bool saved_states, hipStream_t s) {
  const bool d32 = delta_dtype == AK_DTYPE_F32;
  const bool bc32 = bc_dtype == AK_DTYPE_F32;
  if (!d32 && delta_dtype != u_dtype) return -1;
  if (!bc32 && bc_dtype != u_dtype) return -1;
  if (d32 && bc32) launch_scan_bwd<TU, float, float>(p, dB, dC, dA, dD, dbias, saved_states, s);
  else if (d32) launch_scan_bwd<TU, float, TU>(p, dB, dC, dA, dD, dbias, saved_states, s);
  else if (bc32) launch_scan_bwd<TU, TU, float>(p, dB, dC, dA, dD, dbias, saved_states, s);
  else launch_scan_bwd<TU, TU, TU>(p, dB, dC, dA, dD, dbias, saved_states, s);
  return 0;
}

// Checks shared by the forward and backward entry points, and the common
// parameter fields. bc_dtype_eff: the element type of the variable B / C
// (fp32 when both are constant).
int scan_common_args(const char* name, ScanParams& p, int64_t batch, int64_t dim, int64_t seqlen,
                     int64_t dstate, int64_t ngroups, int bc_flags, int u_dtype, int delta_dtype,
                     int bc_dtype, int a_dtype, int* bc_dtype_eff) {
  if (batch < 0 || dim <= 0 || seqlen < 0 || dstate <= 0 || ngroups <= 0)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: bad shape", name);
  if (a_dtype != AK_DTYPE_F32 && a_dtype != AK_DTYPE_C64)
    return ak_set_error(AK_ERR_UNSUPPORTED, "%s: A must be fp32 or complex64", name);
  if (dstate > 256)
    return ak_set_error(AK_ERR_UNSUPPORTED, "%s: dstate=%lld > 256 is not supported", name,
                        (long long)dstate);
  if (bc_flags & ~(AK_SCAN_B_CONST | AK_SCAN_C_CONST))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: unknown bc_flags %d", name, bc_flags);
  if (dim % ngroups) return ak_set_error(AK_ERR_INVALID_ARG, "%s: dim %% ngroups != 0", name);
  const bool both_const = (bc_flags & AK_SCAN_B_CONST) && (bc_flags & AK_SCAN_C_CONST);
  *bc_dtype_eff = both_const ? AK_DTYPE_F32 : bc_dtype;
  if (ak_dtype_size(u_dtype) == 0 || ak_dtype_size(delta_dtype) == 0 ||
      ak_dtype_size(*bc_dtype_eff) == 0)
    return ak_set_error(AK_ERR_UNSUPPORTED, "%s: unsupported dtype", name);
  if (batch > 65535 || dim > (1 << 24) || seqlen > ((int64_t)1 << 31) - kScanT)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: shape too large", name);
  p.batch = (int)batch; p.dim = (int)dim; p.seqlen = (int)seqlen; p.dstate = (int)dstate;
  p.ngroups = (int)ngroups; p.ch_per_group = (int)(dim / ngroups);
  p.tiles_per_group = (p.ch_per_group + kScanCh - 1) / kScanCh;
  if ((int64_t)p.batch * p.ngroups * p.tiles_per_group > 0x7FFFFFFF)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: grid too large", name);
  p.b_const = (bc_flags & AK_SCAN_B_CONST) ? 1 : 0;
  p.c_const = (bc_flags & AK_SCAN_C_CONST) ? 1 : 0;
  p.nchunks = (int)((seqlen + kCk - 1) / kCk);
  p.xchunks = (int)((seqlen + kXChunk - 1) / kXChunk);
  return AK_OK;
}

// B / C strides: variable ([batch, ngroups, dstate, seqlen]) or constant
// ([dim, dstate], group_stride read as the dim stride).
void scan_bc_strides(ScanParams& p, int64_t B_bs, int64_t B_gs, int64_t B_ns, int64_t C_bs,
                     int64_t C_gs, int64_t C_ns) {
  p.B_ns = B_ns;
  p.C_ns = C_ns;
  if (p.b_const) { p.B_bs = 0; p.B_gs = 0; p.B_ds = B_gs; } else { p.B_bs = B_bs; p.B_gs = B_gs; }
  if (p.c_const) { p.C_bs = 0; p.C_gs = 0; p.C_ds = C_gs; } else { p.C_bs = C_bs; p.C_gs = C_gs; }
}

}  // namespace
}  // namespace ak

extern "C" int ak_selective_scan_fwd(
    const void* u, const void* delta, const float* A, const void* B, const void* C,
    const float* D, const void* z, const float* delta_bias, void* out, float* last_state,
    void* out_prez, float* chunk_states, float* checkpoints, int64_t batch, int64_t dim,
    int64_t seqlen, int64_t dstate, int64_t ngroups,
    int64_t u_batch_stride, int64_t u_dim_stride, int64_t delta_batch_stride,
    int64_t delta_dim_stride, int64_t A_dim_stride, int64_t B_batch_stride,
    int64_t B_group_stride, int64_t B_state_stride, int64_t C_batch_stride,
    int64_t C_group_stride, int64_t C_state_stride, int64_t z_batch_stride, int64_t z_dim_stride,
    int64_t out_batch_stride, int64_t out_dim_stride, int delta_softplus, int bc_flags,
    int u_dtype, int delta_dtype, int bc_dtype, int a_dtype, void* stream) {
  const char* name = "ak_selective_scan_fwd";
  ak::ScanParams p{};
  int bc_eff = 0;
  int rc = ak::scan_common_args(name, p, batch, dim, seqlen, dstate, ngroups, bc_flags, u_dtype,
                                delta_dtype, bc_dtype, a_dtype, &bc_eff);
  if (rc) return rc;
  if (batch == 0 || seqlen == 0) return AK_OK;
  if (!u || !delta || !A || !B || !C || !out) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  p.u = u; p.delta = delta; p.A = A; p.B = B; p.C = C; p.D = D; p.z = z;
  p.delta_bias = delta_bias; p.out = out; p.last_state = last_state;
  p.out_prez = out_prez; p.chunk_states = chunk_states;
  p.ck = checkpoints;
  p.u_bs = u_batch_stride; p.u_ds = u_dim_stride; p.d_bs = delta_batch_stride; p.d_ds = delta_dim_stride;
  p.A_ds = A_dim_stride;
  ak::scan_bc_strides(p, B_batch_stride, B_group_stride, B_state_stride, C_batch_stride,
                      C_group_stride, C_state_stride);
  p.z_bs = z_batch_stride; p.z_ds = z_dim_stride; p.o_bs = out_batch_stride; p.o_ds = out_dim_stride;
  p.softplus = delta_softplus ? 1 : 0;
  hipStream_t s = ak_stream(stream);
  if (a_dtype == AK_DTYPE_C64) {
    if (ak::launch_scan_complex_fwd(p, u_dtype, delta_dtype, bc_eff, s))
      return ak_set_error(AK_ERR_UNSUPPORTED, "%s: delta and a variable B/C must be fp32 or the dtype of u", name);
    return ak_check_launch(name);
  }
  bool rows = false;  // dstate in (16, 64]: the specialised kernel with 2 / 4 rows per channel
  if (p.dstate > 16 && p.dstate <= 64) {
    switch (u_dtype) {
      case AK_DTYPE_F32: rows = ak::dispatch_scan_rows<float>(p, u_dtype, delta_dtype, bc_eff, s); break;
      case AK_DTYPE_F16: rows = ak::dispatch_scan_rows<ak::f16>(p, u_dtype, delta_dtype, bc_eff, s); break;
      default: rows = ak::dispatch_scan_rows<ak::bf16>(p, u_dtype, delta_dtype, bc_eff, s); break;
    }
  }
  if (rows) {
    rc = 0;
  } else if (ak::scan_needs_wide(p)) {
    rc = ak::launch_scan_wide_fwd(p, false, u_dtype, delta_dtype, bc_eff, s);
  } else {
    switch (u_dtype) {
      case AK_DTYPE_F32: rc = ak::dispatch_scan<float>(p, u_dtype, delta_dtype, bc_eff, s); break;
      case AK_DTYPE_F16: rc = ak::dispatch_scan<ak::f16>(p, u_dtype, delta_dtype, bc_eff, s); break;
      default: rc = ak::dispatch_scan<ak::bf16>(p, u_dtype, delta_dtype, bc_eff, s); break;
    }
  }
  if (rc) return ak_set_error(AK_ERR_UNSUPPORTED, "%s: delta and a variable B/C must be fp32 or the dtype of u", name);
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
  if (batch * seqlen * d_inner >= ((int64_t)1 << 62)) return ak_set_error(AK_ERR_INVALID_ARG, "%s: shape too large", name);
  const int64_t lanes = batch * d_inner;
  hipStream_t s = ak_stream(stream);
  // chunks when (batch, channel) lanes alone leave the GPU idle (about 2^18
  // lanes in all). Up to 1024 steps one workgroup per 32 channels holds all
  // of a row's chunks (AMADEUS's shape; not below 16 channels, where most of
  // its threads would idle); otherwise the chunked passes, chunks of at most
  // 32 steps in registers, longer ones streaming.
  const int nchunks = ak::diag_chunks(batch, seqlen, d_inner, 18);
  if (nchunks > 1 && seqlen <= ak::kDiagWgLC * ak::kDiagWgLC && d_inner >= ak::kDiagWgCh / 2 &&
      batch * seqlen * d_inner < ((int64_t)1 << 30)) {
    // one launch: every chunk of 32 channels in one workgroup
    const int nck = (int)((seqlen + ak::kDiagWgLC - 1) / ak::kDiagWgLC);
    const int lc = (int)((seqlen + nck - 1) / nck);
    const unsigned grid = (unsigned)(batch * ((d_inner + ak::kDiagWgCh - 1) / ak::kDiagWgCh));
    ak::diag_scan_wg_kernel<<<dim3(grid), dim3(ak::kDiagWgCh * nck), 0, s>>>(
        dA, dBx, C, D, x, y, (int)batch, (int)seqlen, (int)d_inner, lc, nck);
    return ak_check_launch(name);
  }
  if (nchunks <= 1) {
    const unsigned grid = (unsigned)((lanes + 255) / 256);
    ak::diag_scan_kernel<<<dim3(grid), dim3(256), 0, s>>>(dA, dBx, C, D, x, y, (int)batch, (int)seqlen,
                                                         (int)d_inner);
    return ak_check_launch(name);
  }
  const int lc = (int)((seqlen + nchunks - 1) / nchunks);  // >= 16
  const int nc = (int)((seqlen + lc - 1) / lc);             // every chunk but the last is full
  const unsigned g1 = (unsigned)((batch * (nc - 1) * d_inner + 255) / 256);
  const unsigned g2 = (unsigned)((lanes + 255) / 256);
  const unsigned g3 = (unsigned)((batch * nc * d_inner + 255) / 256);
  auto run = [&](auto lc_tag) {
    constexpr int kLC = decltype(lc_tag)::value;
    ak::diag_scan_chunk_agg_kernel<kLC><<<dim3(g1), dim3(256), 0, s>>>(dA, dBx, y, (int)batch, (int)seqlen,
                                                                      (int)d_inner, lc, nc);
    ak::diag_scan_chunk_carry_kernel<<<dim3(g2), dim3(256), 0, s>>>(y, (int)batch, (int)seqlen, (int)d_inner,
                                                                   lc, nc);
    ak::diag_scan_chunk_out_kernel<kLC><<<dim3(g3), dim3(256), 0, s>>>(dA, dBx, C, D, x, y, (int)batch,
                                                                      (int)seqlen, (int)d_inner, lc, nc);
  };
  // (chunks of at most 16 steps arise only for sequences of at most 1024
  // steps, which take the one-launch kernel)
  if (lc <= 32) run(std::integral_constant<int, 32>{});
  else run(std::integral_constant<int, 0>{});
  return ak_check_launch(name);
}

extern "C" size_t ak_diag_scan_bwd_workspace_bytes(int64_t batch, int64_t d_inner) {
  if (batch <= 0 || d_inner <= 0) return 0;
  return (size_t)(((batch * d_inner * 4) + 255) & ~(int64_t)255);
}

extern "C" int ak_diag_scan_bwd(const float* dA, const float* dBx, const float* C, const float* D,
                                const float* x, const float* grad_y, float* grad_dA,
                                float* grad_dBx, float* grad_C, float* grad_D, float* grad_x,
                                void* workspace, size_t workspace_bytes, int64_t batch,
                                int64_t seqlen, int64_t d_inner, void* stream) {
  const char* name = "ak_diag_scan_bwd";
  if (batch < 0 || seqlen < 0 || d_inner <= 0) return ak_set_error(AK_ERR_INVALID_ARG, "%s: bad shape", name);
  if (batch * d_inner > 0x7FFFFFFFll || seqlen > 0x7FFFFFFFll)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: shape too large", name);
  if (!grad_D) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null grad_D", name);
  hipStream_t s = ak_stream(stream);
  if (batch == 0 || seqlen == 0) {
    // no steps: grad_D is a sum over nothing
    ak::diag_scan_gd_kernel<<<dim3((unsigned)((d_inner + 255) / 256)), dim3(256), 0, s>>>(
        nullptr, grad_D, 0, (int)d_inner);
    return ak_check_launch(name);
  }
  if (!dA || !dBx || !C || !D || !x || !grad_y || !grad_dA || !grad_dBx || !grad_C || !grad_x)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  if (!workspace || workspace_bytes < ak_diag_scan_bwd_workspace_bytes(batch, d_inner))
    return ak_set_error(AK_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu", name,
                        workspace_bytes, ak_diag_scan_bwd_workspace_bytes(batch, d_inner));
  float* part = static_cast<float*>(workspace);
  const int64_t lanes = batch * d_inner;
  // Chunks when (batch, channel) lanes alone leave the GPU idle. Up to 1024
  // steps and from 16 channels the workgroup carry kernel and the 32-step
  // sweep (AMADEUS's shape); otherwise the chunked passes, with chunks of at
  // most 32 steps in registers (a plan for about 2^18 lanes) or else
  // streaming (2^17).
  int nc = ak::diag_chunks(batch, seqlen, d_inner, 18);
  int lc = nc > 1 ? (int)((seqlen + nc - 1) / nc) : 0;
  if (nc > 1 && lc > 32) {
    nc = ak::diag_chunks(batch, seqlen, d_inner, 17);
    lc = nc > 1 ? (int)((seqlen + nc - 1) / nc) : 0;
  }
  if (nc > 1) {
    const int ncs = (int)((seqlen + lc - 1) / lc);
    const int B_ = (int)batch, L_ = (int)seqlen, D_ = (int)d_inner;
    const unsigned g_lane = (unsigned)((lanes + 255) / 256);
    const unsigned g_all = (unsigned)((batch * ncs * d_inner + 255) / 256);
    if (seqlen <= ak::kDiagWgLC * ak::kDiagWgLC && d_inner >= ak::kDiagWgCh / 2 &&
        batch * seqlen * d_inner < ((int64_t)1 << 30)) {
      // aggregates and carries in one launch (its own plan: at most 32 chunks
      // of at most 32 steps), then the 32-step sweep on the same chunks
      const int nck = (int)((seqlen + ak::kDiagWgLC - 1) / ak::kDiagWgLC);
      const int lcw = (int)((seqlen + nck - 1) / nck);
      const int ncw = (int)((seqlen + lcw - 1) / lcw);
      const unsigned grid = (unsigned)(batch * ((d_inner + ak::kDiagWgCh - 1) / ak::kDiagWgCh));
      ak::diag_bwd_wg_carry_kernel<<<dim3(grid), dim3(ak::kDiagWgCh * nck), 0, s>>>(
          dA, dBx, C, grad_y, x, grad_dBx, grad_dA, part, B_, L_, D_, lcw, nck);
      const unsigned g_w = (unsigned)((batch * ncw * d_inner + 255) / 256);
      ak::diag_bwd_chunk_kernel<32><<<dim3(g_w), dim3(256), 0, s>>>(
          dA, dBx, C, D, grad_y, grad_dA, grad_dBx, grad_C, grad_x, B_, L_, D_, lcw, ncw);
      ak::diag_scan_gd_kernel<<<dim3((unsigned)((d_inner + 255) / 256)), dim3(256), 0, s>>>(
          part, grad_D, B_, D_);
      return ak_check_launch(name);
    }
    auto run = [&](auto lc_tag) {
      constexpr int kLC = decltype(lc_tag)::value;
      ak::diag_bwd_aggs_kernel<kLC><<<dim3(g_all), dim3(256), 0, s>>>(
          dA, dBx, C, grad_y, x, grad_C, grad_dA, grad_x, grad_dBx, B_, L_, D_, lc, ncs);
      ak::diag_bwd_carries_kernel<<<dim3(g_lane), dim3(256), 0, s>>>(grad_C, grad_dBx, grad_dA, grad_x, part,
                                                                    B_, L_, D_, lc, ncs);
      ak::diag_bwd_chunk_kernel<kLC><<<dim3(g_all), dim3(256), 0, s>>>(
          dA, dBx, C, D, grad_y, grad_dA, grad_dBx, grad_C, grad_x, B_, L_, D_, lc, ncs);
    };
    // (chunks of at most 16 steps arise only for sequences of at most 1024
    // steps, which take the workgroup carry kernel)
    if (lc <= 32) run(std::integral_constant<int, 32>{});
    else run(std::integral_constant<int, 0>{});
    ak::diag_scan_gd_kernel<<<dim3((unsigned)((d_inner + 255) / 256)), dim3(256), 0, s>>>(
        part, grad_D, B_, D_);
    return ak_check_launch(name);
  }
  ak::diag_scan_bwd_kernel<<<dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, s>>>(
      dA, dBx, C, D, x, grad_y, grad_dA, grad_dBx, grad_C, grad_x, part, (int)batch, (int)seqlen,
      (int)d_inner);
  ak::diag_scan_gd_kernel<<<dim3((unsigned)((d_inner + 255) / 256)), dim3(256), 0, s>>>(
      part, grad_D, (int)batch, (int)d_inner);
  return ak_check_launch(name);
}

extern "C" size_t ak_selective_scan_bwd_workspace_bytes(int64_t batch, int64_t dim, int64_t seqlen,
                                                       int64_t dstate, int64_t ngroups,
                                                       int bc_flags) {
  if (batch <= 0 || dim <= 0 || seqlen <= 0 || dstate <= 0 || ngroups <= 0 || dim % ngroups) return 0;
  if (bc_flags & AK_SCAN_A_COMPLEX)
    return ak::scan_complex_bwd_ws(batch, dim, seqlen, dstate, ngroups, bc_flags).total;
  return ak::scan_bwd_ws(batch, dim, seqlen, dstate, ngroups, bc_flags).total;
}

extern "C" int ak_selective_scan_bwd(
    const void* u, const void* delta, const float* A, const void* B, const void* C,
    const float* D, const void* z, const float* delta_bias, const void* dout, void* du,
    void* ddelta, float* dA, void* dB, void* dC, float* dD, void* dz, float* ddelta_bias,
    const float* checkpoints, const void* out_prez,
    void* workspace, size_t workspace_bytes, int64_t batch, int64_t dim, int64_t seqlen,
    int64_t dstate, int64_t ngroups, int64_t u_batch_stride, int64_t u_dim_stride,
    int64_t delta_batch_stride, int64_t delta_dim_stride, int64_t A_dim_stride,
    int64_t B_batch_stride, int64_t B_group_stride, int64_t B_state_stride,
    int64_t C_batch_stride, int64_t C_group_stride, int64_t C_state_stride,
    int64_t z_batch_stride, int64_t z_dim_stride, int64_t dout_batch_stride,
    int64_t dout_dim_stride, int delta_softplus, int bc_flags, int u_dtype, int delta_dtype,
    int bc_dtype, int a_dtype, void* stream) {
  const char* name = "ak_selective_scan_bwd";
  ak::ScanParams p{};
  int bc_eff = 0;
  int rc = ak::scan_common_args(name, p, batch, dim, seqlen, dstate, ngroups, bc_flags, u_dtype,
                                delta_dtype, bc_dtype, a_dtype, &bc_eff);
  if (rc) return rc;
  if (!dA) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null dA", name);
  if (D && !dD) return ak_set_error(AK_ERR_INVALID_ARG, "%s: D given without dD", name);
  if (delta_bias && !ddelta_bias) return ak_set_error(AK_ERR_INVALID_ARG, "%s: delta_bias given without ddelta_bias", name);
  hipStream_t s = ak_stream(stream);
  const bool cplx = a_dtype == AK_DTYPE_C64;
  if (batch == 0 || seqlen == 0) {
    // no steps: dA, dD, ddelta_bias and a constant dB / dC are sums over
    // nothing; a variable dB / dC, du, ... are empty
    if (p.b_const && !dB) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null dB", name);
    if (p.c_const && !dC) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null dC", name);
    if (cplx) {
      ak::launch_scan_complex_zero((int)dim, (int)dstate, dA, dD, ddelta_bias,
                                   p.b_const ? static_cast<float*>(dB) : nullptr,
                                   p.c_const ? static_cast<float*>(dC) : nullptr, s);
      return ak_check_launch(name);
    }
    const ak::FinArgs<float> fa{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                nullptr, dA, p.b_const ? static_cast<float*>(dB) : nullptr,
                                p.c_const ? static_cast<float*>(dC) : nullptr, dD, ddelta_bias, 0,
                                0, 0, (int)dim, (int)dstate};
    ak::scan_bwd_finalize_kernel<float><<<dim3(64), dim3(256), 0, s>>>(fa);
    return ak_check_launch(name);
  }
  if (!u || !delta || !A || !B || !C || !dout || !du || !ddelta || !dB || !dC || (z && !dz))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  if (checkpoints && z && !out_prez)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: checkpoints with a gate z need out_prez", name);
  const ak::ScanBwdWs ws = ak::scan_bwd_ws(batch, dim, seqlen, dstate, ngroups, bc_flags);
  const ak::ZWs zws = ak::scan_complex_bwd_ws(batch, dim, seqlen, dstate, ngroups, bc_flags);
  const size_t need = cplx ? zws.total : ws.total;
  if (!workspace || workspace_bytes < need)
    return ak_set_error(AK_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu", name,
                        workspace_bytes, need);
  p.u = u; p.delta = delta; p.A = A; p.B = B; p.C = C; p.D = D; p.z = z;
  p.delta_bias = delta_bias; p.out = nullptr; p.last_state = nullptr;
  p.u_bs = u_batch_stride; p.u_ds = u_dim_stride; p.d_bs = delta_batch_stride; p.d_ds = delta_dim_stride;
  p.A_ds = A_dim_stride;
  ak::scan_bc_strides(p, B_batch_stride, B_group_stride, B_state_stride, C_batch_stride,
                      C_group_stride, C_state_stride);
  p.z_bs = z_batch_stride; p.z_ds = z_dim_stride;
  p.o_bs = dim * seqlen; p.o_ds = seqlen;  // du, ddelta, dz: contiguous [batch, dim, seqlen]
  p.go_bs = dout_batch_stride; p.go_ds = dout_dim_stride;
  p.softplus = delta_softplus ? 1 : 0;
  p.dout = dout; p.dz = dz; p.du = du; p.ddelta = ddelta;
  if (cplx) {
    p.ck = const_cast<float*>(checkpoints);
    p.out_prez = const_cast<void*>(out_prez);
    if (ak::launch_scan_complex_bwd(p, zws, workspace, checkpoints != nullptr, u_dtype, delta_dtype,
                                    bc_eff, dB, dC, dA, dD, ddelta_bias, s))
      return ak_set_error(AK_ERR_UNSUPPORTED, "%s: delta and a variable B/C must be fp32 or the dtype of u", name);
    return ak_check_launch(name);
  }
  char* w = static_cast<char*>(workspace);
  size_t off = 0;
  auto take = [&](size_t bytes) { float* q = bytes ? reinterpret_cast<float*>(w + off) : nullptr; off += bytes; return q; };
  p.ck = take(ws.ck);
  p.dB_part = take(ws.partB);
  p.dC_part = take(ws.partC);
  p.dA_part = take(ws.dA);
  p.dD_part = take(ws.dD);
  p.dbias_part = take(ws.dD);
  p.dBc_part = take(ws.dBc);
  p.dCc_part = take(ws.dCc);
  // saved forward states: the reverse pass reads them (and out_prez) in place
  if (checkpoints) {
    p.ck = const_cast<float*>(checkpoints);
    p.out_prez = const_cast<void*>(out_prez);
  }
  const bool saved = checkpoints != nullptr;
  if (ak::scan_needs_wide(p)) {
    if (!saved) rc = ak::launch_scan_wide_fwd(p, true, u_dtype, delta_dtype, bc_eff, s);
    if (!rc) rc = ak::launch_scan_wide_bwd(p, u_dtype, delta_dtype, bc_eff, s);
    if (!rc) rc = ak::finish_for(bc_eff, p, dB, dC, dA, dD, ddelta_bias, s);
  } else {
    switch (u_dtype) {
      case AK_DTYPE_F32: rc = ak::dispatch_scan_bwd<float>(p, u_dtype, delta_dtype, bc_eff, dB, dC, dA, dD, ddelta_bias, saved, s); break;
      case AK_DTYPE_F16: rc = ak::dispatch_scan_bwd<ak::f16>(p, u_dtype, delta_dtype, bc_eff, dB, dC, dA, dD, ddelta_bias, saved, s); break;
      default: rc = ak::dispatch_scan_bwd<ak::bf16>(p, u_dtype, delta_dtype, bc_eff, dB, dC, dA, dD, ddelta_bias, saved, s); break;
    }
  }
  if (rc) return ak_set_error(AK_ERR_UNSUPPORTED, "%s: delta and a variable B/C must be fp32 or the dtype of u", name);
  return ak_check_launch(name);
}
