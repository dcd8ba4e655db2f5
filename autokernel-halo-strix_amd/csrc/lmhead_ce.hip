// Fused lm-head GEMM + cross-entropy forward for gfx950.
//
// logits[t, v] = hidden[t, :] . weight[v, :] are produced on the matrix
// cores (v_mfma_f32_32x32x16_{bf16,f16}, fp32 accumulation) and consumed in
// registers: each 256(vocab) x 256(token) workgroup tile reduces its logits
// to one online-softmax partial (max, sum exp(x - max)) per token, and the
// workgroup whose vocab range holds a token's target records that token's
// target logit. Logits never reach memory. A row kernel then merges the
// partials of all vocab tiles into logsumexp and per-token loss, and a
// single-workgroup kernel forms the mean over non-ignored tokens in a fixed
// order (deterministic).
//
// Semantics: kernels/hip/chunked_linear_cross_entropy.py:55-148 and
// kernels/ce_fused.py:236-260 of the reference (loss = lse - logit[target],
// ignored tokens contribute 0 and are excluded from the mean's
// denominator, which is clamped to >= 1). The logsumexp runs over all
// `vocab` columns (padded vocab entries are not masked, as in the reference).
//
// Tile mechanics: the MFMA A operand is a 32-row slab of `weight` (vocab
// rows), B is a 32-row slab of `hidden` (token rows); both are K-contiguous
// in memory and are staged through LDS in 64-wide K steps, double buffered,
// by direct global-to-LDS loads (global_load_lds_dwordx4), with the 16-byte
// chunk index XOR-swizzled by (row / 2) mod 8 so that the ds_read_b128
// fragment reads are bank-conflict free. 4 waves per workgroup (one per SIMD), each owning 128 vocab x 128
// token accumulators (4 x 4 MFMA 32x32 blocks, 256 accumulator registers):
// every 16-byte fragment read from LDS feeds 4 MFMAs, and the fragments of
// the next 16-wide K slice are read while the current slice's 16 MFMAs run. Workgroup ids are remapped so that the 32
// workgroups an XCD runs at once cover a compact 4 x 8 block of tiles and
// share its weight / hidden slabs in that XCD's L2.
#include "ak_common.h"

namespace ak {
namespace {

constexpr int kTV = 256;      // vocab rows per workgroup tile
constexpr int kTT = 256;      // tokens per workgroup tile
constexpr int kKS = 64;       // K per LDS stage
constexpr int kLThreads = 256;
constexpr int kChunks = kKS / 8;                          // 16-byte chunks per staged row
constexpr int kStageChunks = (kTV + kTT) * kChunks;       // u32x4 per stage
constexpr int kGroupV = 4;                                // vocab tiles per XCD group

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16_t mfma32(bf16, u32x4 a, u32x4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma32(f16, u32x4 a, u32x4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

struct MSPair {
  float m, s;
};

template <typename T>
__global__ void __launch_bounds__(kLThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
lmhead_ce_tile_kernel(const T* __restrict__ H, const T* __restrict__ W,
                      const int64_t* __restrict__ targets, MSPair* __restrict__ part,
                      float* __restrict__ tgt_logit, int n_rows, int vocab, int d,
                      int64_t ldh, int64_t ldw, int n_vt, int n_tt) {
  __shared__ u32x4 lds[2 * kStageChunks];  // 128 KiB: two K stages of weight + hidden slabs

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wv = wave >> 1;  // vocab half (128 rows)
  const int wt = wave & 1;   // token half (128 columns)

  // ---- tile coordinates (XCD-grouped order) ----
  const int n_tiles = n_vt * n_tt;
  int lin = blockIdx.x;
  if ((n_tiles & 7) == 0) lin = (lin & 7) * (n_tiles >> 3) + (lin >> 3);
  const int per_group = kGroupV * n_tt;
  const int grp = lin / per_group;
  const int in_grp = lin % per_group;
  const int gv0 = grp * kGroupV;
  const int gvn = min(kGroupV, n_vt - gv0);
  const int vt = gv0 + in_grp % gvn;
  const int tt = in_grp / gvn;
  const int v0 = vt * kTV;
  const int t0 = tt * kTT;

  // ---- global -> LDS loader (direct-to-LDS DMA, no staging registers) ----
  // A stage is 512 rows x 8 chunks of 16 bytes: weight rows 0..255 then
  // hidden rows 256..511. global_load_lds_dwordx4 writes lane i's 16 bytes to
  // (uniform LDS block base + 16 i), so each instruction fills one 1 KiB block
  // = 8 consecutive rows; lane i fetches the logical chunk that the XOR
  // swizzle places at physical chunk i % 8 of row i / 8. Waves 0-1 load the
  // weight slab, waves 2-3 the hidden slab, 128 rows (16 blocks) each.
  const bool loads_w = wave < 2;
  const int lrow0 = (wave & 1) * 128;
  const int first = loads_w ? v0 : t0;
  const int last = (loads_w ? vocab : n_rows) - 1 - first;
  const int64_t gld = loads_w ? ldw : ldh;
  const T* slab = (loads_w ? W : H) + (int64_t)first * gld;
  const int lds_row0 = (loads_w ? 0 : kTV) + lrow0;
  uint32_t goff[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int row = lrow0 + 8 * j + (lane >> 3);
    const int c = (lane & 7) ^ ((row >> 1) & 7);
    goff[j] = (uint32_t)min(row, last) * (uint32_t)gld + 8 * c;
  }
  auto dma = [&](int k0, int st) {
    u32x4* blk = lds + st * kStageChunks + lds_row0 * kChunks;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)(slab + goff[j] + k0),
          (__attribute__((address_space(3))) void*)(blk + 8 * j * kChunks), 16, 0, 0);
    }
  };

  // Fragment reads: rows wv*128 + 32i + lane%32 (weight) and
  // kTV + wt*128 + 32i + lane%32 (hidden); the swizzle is again common to i.
  const int fr = lane & 31;
  const int fsw = (fr >> 1) & 7;
  const int abase = (wv * 128 + fr) * kChunks;
  const int bbase = (kTV + wt * 128 + fr) * kChunks;
  const int khalf = lane >> 5;

  f32x16_t acc[4][4];
#pragma unroll
  for (int vb = 0; vb < 4; ++vb)
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[vb][tb][r] = 0.0f;

  auto load_frags = [&](const u32x4* sb, int kk, u32x4* af, u32x4* bf) {
    const int c = (2 * kk + khalf) ^ fsw;
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = sb[abase + 32 * i * kChunks + c];
#pragma unroll
    for (int i = 0; i < 4; ++i) bf[i] = sb[bbase + 32 * i * kChunks + c];
  };

  // Main loop. Branch-free so the scheduling directives below act on one
  // basic block per K step: the global loads for step ks+1 go out during the
  // first 16-wide slice, each slice's 16 MFMAs are interleaved with the 8
  // ds_reads of the next slice's fragments, and the staged chunks are written
  // to the other LDS stage at the end. On the last step the loader re-reads
  // the last valid K slab into the unused stage instead of branching.
  // Main loop. Branch-free so the scheduling directives below act on one
  // basic block per K step: the DMA for step ks+1 goes out during the first
  // 16-wide slice, and each slice's 16 MFMAs are interleaved with the 8
  // ds_reads of the next slice's fragments. On the last step the loader
  // re-reads the last valid K slab into the unused stage instead of
  // branching. s_waitcnt(0) + barrier publish the new stage.
  const int nk = d / kKS;
  dma(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  u32x4 af[2][4], bf[2][4];
  load_frags(lds, 0, af[0], bf[0]);

  for (int ks = 0; ks < nk; ++ks) {
    const int st = ks & 1;
    const u32x4* sb = lds + st * kStageChunks;
    dma(min(ks + 1, nk - 1) * kKS, st ^ 1);
#pragma unroll
    for (int kk = 0; kk < kKS / 16; ++kk) {
      const int cur = kk & 1;
      if (kk + 1 < kKS / 16) load_frags(sb, kk + 1, af[cur ^ 1], bf[cur ^ 1]);
#pragma unroll
      for (int vb = 0; vb < 4; ++vb)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
          acc[vb][tb] = mfma32(T(), af[cur][vb], bf[cur][tb], acc[vb][tb]);
      if (kk == 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
          __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // 2 global->LDS loads
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
      } else if (kk + 1 < kKS / 16) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    load_frags(lds + (st ^ 1) * kStageChunks, 0, af[0], bf[0]);
  }

  // ---- epilogue: per-token online-softmax partial over this wave's 128 rows ----
  const int vbase = v0 + wv * 128;
  const bool tail = v0 + kTV > vocab;
  float* msbuf = reinterpret_cast<float*>(lds);  // [2 halves][2 (m,s)][256 tokens]
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int col = wt * 128 + tb * 32 + (lane & 31);
    const int tok = t0 + col;
    if (tail) {
#pragma unroll
      for (int vb = 0; vb < 4; ++vb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int v = vbase + vb * 32 + 8 * (r >> 2) + 4 * khalf + (r & 3);
          if (v >= vocab) acc[vb][tb][r] = -INFINITY;
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int vb = 0; vb < 4; ++vb)
#pragma unroll
      for (int r = 0; r < 16; ++r) m = fmaxf(m, acc[vb][tb][r]);
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    const float ms = m * kLog2e;
    float s = 0.0f;
#pragma unroll
    for (int vb = 0; vb < 4; ++vb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += __builtin_amdgcn_exp2f(fmaf(acc[vb][tb][r], kLog2e, -ms));
    s += __shfl_xor(s, 32, 64);

    // target logit: recorded by the one lane that holds it
    if (tok < n_rows) {
      const int64_t tgt = targets[tok];
      const int64_t lr = tgt - vbase;
      if (lr >= 0 && lr < 128 && tgt < vocab) {
        const int i = (int)lr & 31, tvb = (int)lr >> 5;
        if (((i >> 2) & 1) == khalf) {
          const int tr = (i & 3) + 4 * (i >> 3);
          float tv = 0.0f;
#pragma unroll
          for (int vb = 0; vb < 4; ++vb)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              if (vb == tvb && r == tr) tv = acc[vb][tb][r];
          tgt_logit[tok] = tv;
        }
      }
    }
    if (lane < 32) {
      msbuf[(wv * 2 + 0) * kTT + col] = m;
      msbuf[(wv * 2 + 1) * kTT + col] = s;
    }
  }
  __syncthreads();
  // merge the two vocab halves and publish this tile's partial
  {
    const int tok = t0 + tid;
    if (tok < n_rows) {
      const float m0 = msbuf[0 * kTT + tid], s0 = msbuf[1 * kTT + tid];
      const float m1 = msbuf[2 * kTT + tid], s1 = msbuf[3 * kTT + tid];
      const float m = fmaxf(m0, m1);
      float s = 0.0f;
      if (m0 != -INFINITY) s += s0 * __builtin_amdgcn_exp2f((m0 - m) * kLog2e);
      if (m1 != -INFINITY) s += s1 * __builtin_amdgcn_exp2f((m1 - m) * kLog2e);
      part[(int64_t)vt * n_rows + tok] = MSPair{m, s};
    }
  }
}

// lse / per-token loss from the vocab-tile partials. A 1024-thread workgroup
// owns 64 tokens; its 16 waves each fold every 16th vocab tile with an online
// (max, sum) merge (coalesced 512-byte reads per wave), then the 16 partial
// states are merged in a fixed order through LDS (deterministic).
constexpr int kRowsPerBlock = 64;
constexpr int kRowGroups = 16;

__device__ __forceinline__ MSPair ms_merge(MSPair a, MSPair b) {
  const float m = fmaxf(a.m, b.m);
  if (m == -INFINITY) return {m, 0.0f};
  float s = 0.0f;
  if (a.m != -INFINITY) s += a.s * __builtin_amdgcn_exp2f((a.m - m) * kLog2e);
  if (b.m != -INFINITY) s += b.s * __builtin_amdgcn_exp2f((b.m - m) * kLog2e);
  return {m, s};
}

__global__ void __launch_bounds__(kRowsPerBlock * kRowGroups)
lmhead_ce_rows_kernel(const MSPair* __restrict__ part, const float* __restrict__ tgt_logit,
                      const int64_t* __restrict__ targets, float* __restrict__ lse,
                      float* __restrict__ losses, int n_rows, int vocab, int n_vt,
                      int64_t ignore_index) {
  __shared__ MSPair red[kRowGroups][kRowsPerBlock];
  const int r = threadIdx.x % kRowsPerBlock;
  const int grp = threadIdx.x / kRowsPerBlock;
  const int row = blockIdx.x * kRowsPerBlock + r;
  MSPair st{-INFINITY, 0.0f};
  if (row < n_rows) {
#pragma unroll 4
    for (int v = grp; v < n_vt; v += kRowGroups) st = ms_merge(st, part[(int64_t)v * n_rows + row]);
  }
  red[grp][r] = st;
  __syncthreads();
  if (grp != 0 || row >= n_rows) return;
  for (int g = 1; g < kRowGroups; ++g) st = ms_merge(st, red[g][r]);
  const float l = st.m + fast_log(st.s);
  lse[row] = l;
  const int64_t t = targets[row];
  float loss;
  if (t == ignore_index) loss = 0.0f;
  else if (t < 0 || t >= vocab) loss = NAN;
  else loss = l - tgt_logit[row];
  losses[row] = loss;
}

// mean over non-ignored tokens, fixed summation order (one workgroup).
__global__ void __launch_bounds__(1024)
lmhead_ce_mean_kernel(const float* __restrict__ losses, const int64_t* __restrict__ targets,
                      float* __restrict__ loss_out, int64_t* __restrict__ n_valid_out, int n_rows,
                      int64_t ignore_index) {
  float sum = 0.0f;
  int cnt = 0;
  for (int i = threadIdx.x; i < n_rows; i += 1024) {
    sum += losses[i];
    cnt += targets[i] != ignore_index;
  }
  sum = wave_sum(sum);
  float fc = wave_sum((float)cnt);
  __shared__ float ss[16], sc[16];
  if ((threadIdx.x & 63) == 0) {
    ss[threadIdx.x >> 6] = sum;
    sc[threadIdx.x >> 6] = fc;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float tot = 0.0f, c = 0.0f;
    for (int w = 0; w < 16; ++w) {
      tot += ss[w];
      c += sc[w];
    }
    loss_out[0] = tot / fmaxf(c, 1.0f);
    if (n_valid_out) n_valid_out[0] = (int64_t)c;
  }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct WsLayout {
  size_t part, tgt, losses, total;
};

WsLayout ws_layout(int64_t n_rows, int64_t vocab) {
  const int64_t n_vt = (vocab + kTV - 1) / kTV;
  WsLayout w;
  w.part = 0;
  w.tgt = align256((size_t)n_vt * n_rows * sizeof(MSPair));
  w.losses = w.tgt + align256((size_t)n_rows * 4);
  w.total = w.losses + align256((size_t)n_rows * 4);
  return w;
}

template <typename T>
void launch_lmhead(const void* h, const void* w, const int64_t* targets, float* loss, float* lse,
                   float* losses, int64_t* n_valid, void* ws, int n_rows, int vocab, int d,
                   int64_t ldh, int64_t ldw, int64_t ignore_index, hipStream_t s) {
  const int n_vt = (vocab + kTV - 1) / kTV;
  const int n_tt = (n_rows + kTT - 1) / kTT;
  WsLayout L = ws_layout(n_rows, vocab);
  char* base = static_cast<char*>(ws);
  MSPair* part = reinterpret_cast<MSPair*>(base + L.part);
  float* tgt = reinterpret_cast<float*>(base + L.tgt);
  float* lrow = losses ? losses : reinterpret_cast<float*>(base + L.losses);
  lmhead_ce_tile_kernel<T><<<dim3(n_vt * n_tt), dim3(kLThreads), 0, s>>>(
      static_cast<const T*>(h), static_cast<const T*>(w), targets, part, tgt, n_rows, vocab, d, ldh,
      ldw, n_vt, n_tt);
  lmhead_ce_rows_kernel<<<dim3((n_rows + kRowsPerBlock - 1) / kRowsPerBlock),
                          dim3(kRowsPerBlock * kRowGroups), 0, s>>>(
      part, tgt, targets, lse, lrow, n_rows, vocab, n_vt, ignore_index);
  lmhead_ce_mean_kernel<<<dim3(1), dim3(1024), 0, s>>>(lrow, targets, loss, n_valid, n_rows,
                                                      ignore_index);
}

}  // namespace
}  // namespace ak

extern "C" size_t ak_lmhead_ce_workspace_bytes(int64_t n_rows, int64_t vocab) {
  if (n_rows <= 0 || vocab <= 0) return 0;
  return ak::ws_layout(n_rows, vocab).total;
}

extern "C" int ak_lmhead_ce_fwd(const void* hidden, const void* weight, const int64_t* targets,
                                float* loss, float* lse, float* losses, int64_t* n_valid,
                                void* workspace, size_t workspace_bytes, int64_t n_rows,
                                int64_t vocab, int64_t d, int64_t ld_h, int64_t ld_w,
                                int64_t ignore_index, int dtype, void* stream) {
  const char* name = "ak_lmhead_ce_fwd";
  if (dtype != AK_DTYPE_BF16 && dtype != AK_DTYPE_F16)
    return ak_set_error(AK_ERR_UNSUPPORTED, "%s: dtype must be bf16 or fp16", name);
  if (n_rows <= 0 || vocab <= 0 || d <= 0)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: bad shape n_rows=%lld vocab=%lld d=%lld", name,
                        (long long)n_rows, (long long)vocab, (long long)d);
  if (d % ak::kKS) return ak_set_error(AK_ERR_UNSUPPORTED, "%s: d=%lld must be a multiple of %d", name, (long long)d, ak::kKS);
  if (n_rows > (1 << 30) || vocab > (1 << 30) || d > (1 << 20))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: shape too large", name);
  if (ld_h < d || ld_w < d || ld_h % 8 || ld_w % 8)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: row pitches must be >= d and multiples of 8 elements", name);
  if (!hidden || !weight || !targets || !loss || !lse || !workspace)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  if (!ak::aligned16(hidden) || !ak::aligned16(weight) || !ak::aligned16(workspace))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: hidden, weight and workspace must be 16-byte aligned", name);
  const int64_t n_tiles = ((vocab + ak::kTV - 1) / ak::kTV) * ((n_rows + ak::kTT - 1) / ak::kTT);
  if (n_tiles > 0x7FFFFFFF) return ak_set_error(AK_ERR_INVALID_ARG, "%s: too many tiles", name);
  if (workspace_bytes < ak::ws_layout(n_rows, vocab).total)
    return ak_set_error(AK_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu", name,
                        workspace_bytes, ak::ws_layout(n_rows, vocab).total);
  hipStream_t s = ak_stream(stream);
  if (dtype == AK_DTYPE_BF16)
    ak::launch_lmhead<ak::bf16>(hidden, weight, targets, loss, lse, losses, n_valid, workspace,
                                (int)n_rows, (int)vocab, (int)d, ld_h, ld_w, ignore_index, s);
  else
    ak::launch_lmhead<ak::f16>(hidden, weight, targets, loss, lse, losses, n_valid, workspace,
                               (int)n_rows, (int)vocab, (int)d, ld_h, ld_w, ignore_index, s);
  return ak_check_launch(name);
}
