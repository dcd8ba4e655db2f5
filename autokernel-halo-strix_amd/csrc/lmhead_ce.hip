// Fused lm-head GEMM + cross-entropy forward for gfx950.
//
// logits[t, v] = hidden[t, :] . weight[v, :] are produced on the matrix
// cores (v_mfma_f32_32x32x16_{bf16,f16}, fp32 accumulation) and consumed in
// registers: each wave of a 256(vocab) x 256(token) tile reduces its
// 128 x 128 block of logits to one online-softmax partial (max, sum
// exp(x - max)) per token. Logits never reach memory. A row kernel then
// merges the partials of all vocab tiles into logsumexp, computes each
// token's target logit as its own dot product hidden[t] . weight[target[t]]
// (fp32 accumulation) and forms the per-token loss; a single-workgroup
// kernel forms the mean over non-ignored tokens in a fixed order
// (deterministic).
//
// Semantics: kernels/hip/chunked_linear_cross_entropy.py:55-148 and
// kernels/ce_fused.py:236-260 of the reference (loss = lse - logit[target],
// ignored tokens contribute 0 and are excluded from the mean's
// denominator, which is clamped to >= 1). The logsumexp runs over all
// `vocab` columns (padded vocab entries are not masked, as in the reference).
// Options: a logit softcap z' = cap tanh(z / cap), and label smoothing a
// (loss = lse - (1 - a) z'_t - a mean(z'); the tile kernel then also writes
// per-partial sums of z', merged by the row kernel in a fixed order).
//
// Tile kernel mechanics:
// * Persistent: one 256-thread workgroup per CU walks its tiles in an
//   XCD-grouped order (the 32 workgroups of an XCD cover a compact block of
//   vocab x token tiles, so their weight / hidden slabs are shared in that
//   XCD's L2).
// * Operands: the MFMA A operand is a 32-row slab of `weight` (vocab rows),
//   B a 32-row slab of `hidden` (token rows). Both are K-contiguous and are
//   staged through LDS in K blocks of 64 (one 128-byte cache line per row)
//   by direct global-to-LDS loads (global_load_lds_dwordx4, 8 rows x 128 B
//   per instruction). The 160 KiB of LDS hold a ring of 5 slots of 256 rows
//   x 128 B; weight and hidden blocks take turns, each operand is loaded
//   two K blocks ahead of its use, and the loads are spread over the block's
//   MFMAs so that the CU's address unit keeps up without stalling them. The
//   ring runs on across tile boundaries. The 16-byte chunk index of a staged row is XOR-swizzled by
//   (row / 2) mod 8, which makes the ds_read_b128 fragment reads
//   bank-conflict free.
// * 4 waves (one per SIMD), each owning 128 vocab x 128 token accumulators
//   (4 x 4 MFMA 32x32 blocks, 256 accumulator registers): every 16-byte
//   fragment read from LDS feeds 4 MFMAs. The instruction order is pinned:
//   the 16 MFMAs of a 16-wide K slice run over 16 different accumulators
//   while the fragments of the slice after next are read; one barrier per K
//   block (after its second slice) publishes the next block's slots.
#include "mfma_ring.h"

namespace ak {
namespace {

constexpr int kTV = 256;      // vocab rows per tile
constexpr int kTT = 256;      // tokens per tile
constexpr int kLThreads = 256;
constexpr int kGroupV = 4;                               // vocab tiles per XCD group

struct MSPair {
  float m, s;
};

// Tile coordinates of this workgroup's i-th tile. Work item w = block + i *
// grid runs on XCD w % 8 (workgroups are dealt to the 8 XCDs round-robin);
// items of one XCD are numbered consecutively, then cut into groups of
// kGroupV vocab tiles x all token tiles, token-minor within a group.
__device__ __forceinline__ void tile_coords(int i, int n_vt, int n_tt, int& vt, int& tt) {
  const int n_tiles = n_vt * n_tt;
  const int w = (int)blockIdx.x + i * (int)gridDim.x;
  int lin = w;
  if ((gridDim.x & 7) == 0) {
    const int x = w & 7, base = n_tiles >> 3, rem = n_tiles & 7;
    lin = x * base + min(x, rem) + (w >> 3);
  }
  const int per_group = kGroupV * n_tt;
  const int grp = lin / per_group;
  const int in_grp = lin - grp * per_group;
  const int gv0 = grp * kGroupV;
  const int gvn = min(kGroupV, n_vt - gv0);
  vt = gv0 + in_grp % gvn;
  tt = in_grp / gvn;
}

// Instruction order of one 16-MFMA K slice: kDs x (MFMA, DS read), then
// kDmaN x (MFMA, global-to-LDS load), then the remaining MFMAs. (Finer
// interleavings are not honoured by the compiler's scheduler, which then
// clusters the reads.)
template <int kDs, int kDmaN>
__device__ __forceinline__ void slice_order() {
#pragma unroll
  for (int i = 0; i < kDs; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
  }
#pragma unroll
  for (int i = 0; i < kDmaN; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // 1 global->LDS load
  }
  if (16 - kDs - kDmaN > 0) __builtin_amdgcn_sched_group_barrier(0x008, 16 - kDs - kDmaN, 0);
  __builtin_amdgcn_sched_barrier(0);
}

// Row range of a tile along one dimension of `n` rows: the tile owns rows
// [own, min(own + 256, n)) and stages the 256 rows starting at `first`. With
// kShift (n >= 256) a tail tile is shifted back so that its 256 staged rows
// end at row n - 1 (the overlap with the previous tile is masked);
// otherwise staged rows past n - 1 re-read row n - 1.
template <bool kShift>
__device__ __forceinline__ int tile_first(int own, int n) {
  return kShift ? min(own, n - 256) : own;
}

// Backward (kGrad) outputs: dz[t, v] = (softmax(logits)[t, v] - a / vocab) * s_t
// (a = label smoothing, and times 1 - tanh^2 under a softcap) with
// s_t = grad_loss / denom for a counted token, 0 for an ignored one and NaN
// for a target outside [0, vocab); the target entry itself is written
// afterwards by lmhead_ce_grad_target_kernel.
struct GradArgs {
  const float* lse;        // [n_rows] logsumexp of the forward
  const int64_t* targets;  // [n_rows]
  const float* grad_loss;  // [1] upstream gradient of the mean loss
  const float* denom;      // [1] number of counted tokens (clamped >= 1)
  void* dz;                // [n_rows, ld_dz] element type T
  int64_t ld_dz;
  int64_t ignore_index;
  float cap;               // logit softcap (> 0 with kCap; the forward uses it too)
  float ls;                // label smoothing alpha (0 = off)
  float* zsum;             // forward with label smoothing: per-partial sums of the logits
  // backward over a vocab range: the kernels see the weight rows [v0, v0 +
  // vocab) as a vocab of their own; targets and a / vocab refer to the full
  // vocabulary of vocab_total entries
  int64_t v0;
  int64_t vocab_total;
};

// Logit softcap z' = cap * tanh(z / cap), evaluated without cancellation
// through q = exp(2 z / cap) and r = 1 / (q + 1):
//   z' - cap = -2 cap r,   1 - tanh^2 = 4 q r^2.
// k2 = 2 log2(e) / cap and nc = -2 cap log2(e) are per-call constants.
struct Cap {
  float k2, nc;
  __device__ __forceinline__ explicit Cap(float cap) : k2(2.0f * kLog2e / cap), nc(-2.0f * cap * kLog2e) {}
  __device__ __forceinline__ float q(float z) const { return __builtin_amdgcn_exp2f(z * k2); }
};

// Partial of vocab tile vt, vocab half h (0/1), token t: part[(2 vt + h) * n_rows + t].
//
// kFineMask: the vocab rows a tile owns may end inside a wave's 128-row
// half (vocab % 128 != 0, or unshifted tail tiles), so the epilogue masks
// element by element; otherwise a wave's half is either wholly owned or
// wholly skipped.
// kCap: logit softcap ga.cap. The forward partial of a tile is then (cap,
// sum exp(z' - cap)): z' <= cap, so no max pass is needed.
// kLs (forward): label smoothing; the tile also writes the sum of its (capped)
// logits per token to ga.zsum, laid out as the partials. A template flag, so
// that the kernels without it carry no extra register pressure.
template <typename T, bool kShift, bool kFineMask, bool kGrad, bool kCap = false, bool kLs = false>
__global__ void __launch_bounds__(kLThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
lmhead_ce_tile_kernel(const T* __restrict__ H, const T* __restrict__ W, MSPair* __restrict__ part,
                      int n_rows, int vocab, int d, int64_t ldh, int64_t ldw, int n_vt, int n_tt,
                      GradArgs ga) {
  __shared__ u32x4 lds[kSlots * kSlotChunks];  // 160 KiB ring

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wv = wave >> 1;  // vocab half (128 rows) of the accumulators
  const int wt = wave & 1;   // token half (128 columns)

  const int n_tiles = n_vt * n_tt;
  const int n_my = (int)blockIdx.x < n_tiles ? (n_tiles - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
  if (n_my == 0) return;
  const int nb = d / kKB;  // K blocks per tile

  // ---- loader ----
  // A slot is 256 rows x 8 chunks of 16 bytes. global_load_lds_dwordx4
  // writes lane i's 16 bytes to (uniform LDS base + 16 i), so one
  // instruction fills 8 consecutive rows, each a full 128-byte line; lane i
  // fetches the logical chunk that the swizzle puts at physical chunk i % 8
  // of row i / 8. Each wave stages 64 rows of every slot. Byte offsets
  // within a 256-row slab fit 32 bits (row pitch < 2^23 elements).
  // The row of instruction j is lrow + 8 j; its swizzle key ((row / 2) mod
  // 8) = (4 j + lane / 16) mod 8 depends on j only through j's parity.
  const int lrow = wave * 64 + (lane >> 3);
  const uint32_t c16[2] = {16u * (uint32_t)((lane & 7) ^ (lane >> 4)),
                           16u * (uint32_t)((lane & 7) ^ ((lane >> 4) + 4))};
  const uint32_t ldw_b = (uint32_t)ldw * (uint32_t)sizeof(T);
  const uint32_t ldh_b = (uint32_t)ldh * (uint32_t)sizeof(T);
  const uint32_t voff_w[2] = {(uint32_t)lrow * ldw_b + c16[0], (uint32_t)lrow * ldw_b + c16[1]};
  const uint32_t voff_h[2] = {(uint32_t)lrow * ldh_b + c16[0], (uint32_t)lrow * ldh_b + c16[1]};
  // Where the rows of one operand of one K block come from.
  struct Src {
    const char* p;  // row 0 of the 256-row slab, at the block's K offset
    int last;       // last valid slab row (clamped variant only)
  };
  auto dma = [&](Src src, uint32_t ld_b, const uint32_t* voff, int slot, int j0 = 0,
                 int j1 = kDma) {
    u32x4* blk = lds + slot * kSlotChunks + wave * 64 * kChunks;
#pragma unroll
    for (int j = j0; j < j1; ++j) {
      const char* q;
      if (kShift) q = src.p + 8 * j * ld_b + voff[j & 1];
      else q = src.p + (uint32_t)min(lrow + 8 * j, src.last) * ld_b + c16[j & 1];
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)q,
                                       (__attribute__((address_space(3))) void*)(blk + 8 * j * kChunks),
                                       16, 0, 0);
    }
  };
  // Cursor over (tile, K block) for one operand: the slab of this
  // workgroup's tile `it` (tiles past the last one repeat the last tile).
  struct Cursor {
    int it, blk;
    const char* slab;
    int last;
  };
  auto cursor_tile = [&](Cursor& c, bool is_w) {
    int vt, tt;
    tile_coords(min(c.it, n_my - 1), n_vt, n_tt, vt, tt);
    const int n = is_w ? vocab : n_rows;
    const int first = tile_first<kShift>(is_w ? vt * kTV : tt * kTT, n);
    c.slab = reinterpret_cast<const char*>((is_w ? W : H) + (int64_t)first * (is_w ? ldw : ldh));
    c.last = n - 1 - first;
  };
  auto cursor_src = [&](const Cursor& c) {
    return Src{c.slab + c.blk * kKB * (int)sizeof(T), c.last};
  };
  auto cursor_next = [&](Cursor& c, bool is_w) {
    if (++c.blk == nb) {
      c.blk = 0;
      ++c.it;
      cursor_tile(c, is_w);
    }
  };

  // ---- fragment reads ----
  // Rows wv*128 + 32i + lane%32 of the weight slot and wt*128 + 32i +
  // lane%32 of the hidden slot; lanes 32-63 take the upper 8 K of a slice.
  const int fr = lane & 31;
  const int fsw = (fr >> 1) & 7;
  const int khalf = lane >> 5;
  const int arow = (wv * 128 + fr) * kChunks;
  const int brow = (wt * 128 + fr) * kChunks;
  auto frag = [&](int slot, int row, int i, int kk) {
    return lds[slot * kSlotChunks + row + 32 * i * kChunks + ((2 * kk + khalf) ^ fsw)];
  };

  // ---- prologue: K blocks 0 and 1 ----
  // Ring order: W0 H0 W1 H1 W2 H2 W3 ...; operand block q lives in slot q % 5.
  Cursor cw{0, 0, nullptr, 0}, ch{0, 0, nullptr, 0};
  cursor_tile(cw, true);
  cursor_tile(ch, false);
  dma(cursor_src(cw), ldw_b, voff_w, 0);  // q = 0
  cursor_next(cw, true);
  dma(cursor_src(ch), ldh_b, voff_h, 1);  // q = 1
  cursor_next(ch, false);
  dma(cursor_src(cw), ldw_b, voff_w, 2);  // q = 2
  dma(cursor_src(ch), ldh_b, voff_h, 3);  // q = 3
  // cw and ch at K block 1: each K block first advances them to the blocks
  // it loads (weight and hidden of block j + 2)
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(2 * kDma));  // q = 0, 1 landed
  ring_barrier();

  f32x16_t acc[4][4];
  u32x4 af[4][4], bf[4][4];  // fragments of the 4 slices of a K block

  // Slots of K block j (counted over all of this workgroup's blocks):
  // weight in (2j) % 5, hidden in (2j + 1) % 5.
  int sw = 0, sh = 1;
  auto load_frags = [&](int slw, int slh, int kk, u32x4* a, u32x4* b) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = frag(slw, arow, i, kk);
      b[i] = frag(slh, brow, i, kk);
    }
  };
  auto mfmas = [&](auto first_tag, const u32x4* a, const u32x4* b) {
    constexpr bool kFirst = decltype(first_tag)::value;
#pragma unroll
    for (int vb = 0; vb < 4; ++vb)
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
        acc[vb][tb] = mfma32(T(), a[vb], b[tb], kFirst ? f32x16_t{} : acc[vb][tb]);
  };

  // One K block j: 4 slices of 16 MFMAs. Fragments are read two slices
  // ahead of their MFMAs (slices 0 and 1 of block j are in af/bf[0..1] on
  // entry), which gives the LDS reads a full slice of slack against the
  // ring's DMA writes into LDS. Loads are spread over the block so that the
  // CU's address unit (about 20 cycles per 1 KiB load) is never asked for
  // more than a slice can cover: the weight operand of block j + 2 goes into
  // slot (2j + 4) % 5 (free since block j - 1) during slices 0 and 1. The
  // barrier after slice 1 (a) shows every wave done reading block j's slots
  // (its last fragments are read during slice 1), and the hidden operand of
  // block j + 2 then goes into block j's weight slot during slices 2 and 3;
  // (b) publishes block j + 1's slots, whose first two slices' fragments
  // slices 2 and 3 read (this wave's loads of them are done once only the 8
  // loads issued after them, weight j + 2, are outstanding; memory
  // operations complete in issue order, and anything else issued later only
  // makes the wait stricter). A tile's last block reads no fragments of the
  // next block (the epilogue runs first).
  auto block = [&](auto first_tag, auto last_tag) {
    constexpr bool kLastBlk = decltype(last_tag)::value;
    cursor_next(cw, true);
    cursor_next(ch, false);
    const Src ws = cursor_src(cw), hs = cursor_src(ch);
    const int pw = sw + 4 >= kSlots ? sw + 4 - kSlots : sw + 4;  // slot of q = 2j + 4
    const int nsw = sw + 2 >= kSlots ? sw + 2 - kSlots : sw + 2;
    const int nsh = sh + 2 >= kSlots ? sh + 2 - kSlots : sh + 2;
    load_frags(sw, sh, 2, af[2], bf[2]);
    mfmas(first_tag, af[0], bf[0]);
    dma(ws, ldw_b, voff_w, pw, 0, kDma / 2);
    slice_order<8, kDma / 2>();
    load_frags(sw, sh, 3, af[3], bf[3]);
    mfmas(std::false_type{}, af[1], bf[1]);
    dma(ws, ldw_b, voff_w, pw, kDma / 2, kDma);
    slice_order<8, kDma / 2>();
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(kDma));
    ring_barrier();
    if (!kLastBlk) load_frags(nsw, nsh, 0, af[0], bf[0]);
    mfmas(std::false_type{}, af[2], bf[2]);
    dma(hs, ldh_b, voff_h, sw, 0, kDma / 2);
    if constexpr (kLastBlk) slice_order<0, kDma / 2>();
    else slice_order<8, kDma / 2>();
    if (!kLastBlk) load_frags(nsw, nsh, 1, af[1], bf[1]);
    mfmas(std::false_type{}, af[3], bf[3]);
    dma(hs, ldh_b, voff_h, sw, kDma / 2, kDma);
    if constexpr (kLastBlk) slice_order<0, kDma / 2>();
    else slice_order<8, kDma / 2>();
    sw = nsw;
    sh = nsh;
  };

  using yes = std::true_type;
  using no = std::false_type;
  // backward: upstream gradient / number of counted tokens, read once
  const float gs = kGrad ? ga.grad_loss[0] / ga.denom[0] : 0.0f;
  for (int it = 0; it < n_my; ++it) {
    int vt, tt;
    tile_coords(it, n_vt, n_tt, vt, tt);
    const int v_own = vt * kTV, t_own = tt * kTT;
    const int v_first = tile_first<kShift>(v_own, vocab);
    const int t_first = tile_first<kShift>(t_own, n_rows);

    load_frags(sw, sh, 0, af[0], bf[0]);
    load_frags(sw, sh, 1, af[1], bf[1]);
    // backward: the tile's logsumexp and targets, loaded before its last K
    // block. Vector-memory operations complete in issue order, so a load
    // issued in the epilogue would wait for the ring's DMA and the previous
    // tile's dlogits stores as well; issued here, only the last block's DMA
    // is behind it.
    float pre_lse[4];
    int64_t pre_tg[4];
    auto prefetch_rows = [&]() {
      if constexpr (kGrad) {
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          const int tok_c = min(t_first + wt * 128 + tb * 32 + fr, n_rows - 1);
          pre_lse[tb] = ga.lse[tok_c];
          pre_tg[tb] = ga.targets[tok_c];
        }
      }
    };
    if (nb == 1) {
      prefetch_rows();
      block(yes{}, yes{});
    } else {
      block(yes{}, no{});
      for (int kb = 1; kb < nb - 1; ++kb) block(no{}, no{});
      prefetch_rows();
      block(no{}, yes{});
    }
    // The epilogue reads the accumulators with explicit v_accvgpr_read
    // instructions, which the compiler does not space from the last MFMAs
    // that wrote them: give those MFMAs (16 passes at most) their wait states.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");

    // ---- epilogue: per-token online-softmax partial of this wave's 128 rows ----
    // Row x of this wave's 128-row half (counted from its first staged row,
    // lanes 32-63 offset by 4) is a real, owned vocab entry iff lo <= x < hi.
    const int lo_w = v_own - v_first - wv * 128;                    // wave-uniform
    const int hi_w = min(vocab, v_own + kTV) - v_first - wv * 128;
    const int lo = lo_w - 4 * khalf;
    const int hi = hi_w - 4 * khalf;
    if constexpr (kGrad) {
      // dz = exp(z - lse_t) * s_t for this wave's 128 vocab rows x 128
      // tokens. A lane holds token t_first + wt*128 + tb*32 + lane%32 and, per
      // 32-row vocab block, rows 8g + 4*khalf + 0..3 (g = 0..3) of that token.
      // v_permlane32_swap pairs groups (0, 2) and (1, 3) across the two half
      // waves, so that every lane then holds 8 consecutive vocab entries of one
      // token row: one 16-byte store (kFineMask: element-wise stores).
      T* dzp = static_cast<T*>(ga.dz);
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const int tok = t_first + wt * 128 + tb * 32 + fr;
        const int tok_c = min(tok, n_rows - 1);
        const bool tok_ok = tok >= t_own && tok < n_rows;
        const float lse2 = pre_lse[tb] * kLog2e;
        const float cl2 = kCap ? ga.cap * kLog2e - lse2 : 0.0f;  // log2 of exp(cap - lse)
        const int64_t tg = pre_tg[tb];
        const float st = tg == ga.ignore_index ? 0.0f : ((tg < 0 || tg >= ga.vocab_total) ? NAN : gs);
        const float nls = -(ga.ls / (float)ga.vocab_total) * st;  // label smoothing's uniform term
        T* drow = dzp + (int64_t)tok_c * ga.ld_dz + v_first + wv * 128;
#pragma unroll
        for (int vb = 0; vb < 4; ++vb) {
          uint32_t pk[4][2];
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            float e[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float z = acc_read(acc[vb][tb][4 * g4 + j]);
              if constexpr (kCap) {
                // softmax(z')_v * s_t * dz'/dz
                const Cap cp(ga.cap);
                const float q = cp.q(z);
                const float r = __builtin_amdgcn_rcpf(q + 1.0f);
                const float p = __builtin_amdgcn_exp2f(fmaf(cp.nc, r, cl2));
                e[j] = fmaf(p, st, nls) * (4.0f * q * r * r);
              } else {
                e[j] = fmaf(__builtin_amdgcn_exp2f(fmaf(z, kLog2e, -lse2)), st, nls);
              }
            }
            const int x0 = vb * 32 + 8 * g4;  // row of e[0] in the half, as counted by lo / hi
            if constexpr (kFineMask) {
#pragma unroll
              for (int j = 0; j < 4; ++j)
                if (tok_ok && x0 + j >= lo && x0 + j < hi) drow[4 * khalf + x0 + j] = from_f32<T>(e[j]);
            } else {
#pragma unroll
              for (int j = 0; j < 2; ++j) pk[g4][j] = pack2<T>(e[2 * j], e[2 * j + 1]);
            }
          }
          if constexpr (!kFineMask) {
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) {
              // lanes 0-31 end with rows 0..7 of group pr, lanes 32-63 with
              // rows 0..7 of group pr + 2, both as (x0, x1, y0, y1)
              const auto s0 = __builtin_amdgcn_permlane32_swap(pk[pr][0], pk[pr + 2][0], false, false);
              const auto s1 = __builtin_amdgcn_permlane32_swap(pk[pr][1], pk[pr + 2][1], false, false);
              const int x0 = vb * 32 + 8 * (pr + 2 * khalf);
              if (tok_ok && x0 >= lo_w && x0 < hi_w) {
                const u32x4 v = {s0[0], s1[0], s0[1], s1[1]};
                *reinterpret_cast<u32x4*>(drow + x0) = v;
              }
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      continue;
    }
    MSPair* prow = part + (int64_t)(2 * vt + wv) * n_rows;
    MSPair res[4];
    float zres[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // label smoothing: sums of the (capped) logits
    auto epilogue = [&](auto tail_tag) {
      constexpr bool kTail = decltype(tail_tag)::value;
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        // this token block's 64 logits of the lane, read once from the AGPRs
        float x[4][16];
#pragma unroll
        for (int vb = 0; vb < 4; ++vb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            x[vb][r] = acc_read(acc[vb][tb][r]);
            if (kTail) {
              const int o = vb * 32 + 8 * (r >> 2) + (r & 3);
              x[vb][r] = (o >= lo && o < hi) ? x[vb][r] : -INFINITY;
            }
          }
        if constexpr (kCap) {
          // (cap, sum exp(z' - cap)) with exp(z' - cap) = exp2(nc r); masked
          // rows (x = -inf) would give exp(-2 cap) and are dropped. With label
          // smoothing the capped logits z' = cap - 2 cap r are summed too.
          const Cap cp(ga.cap);
          float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f}, z4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int vb = 0; vb < 4; ++vb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float rr = __builtin_amdgcn_rcpf(cp.q(x[vb][r]) + 1.0f);
              const bool live = !(kTail && x[vb][r] == -INFINITY);
              s4[r & 3] += live ? __builtin_amdgcn_exp2f(cp.nc * rr) : 0.0f;
              if constexpr (kLs) z4[r & 3] += live ? fmaf(-2.0f * ga.cap, rr, ga.cap) : 0.0f;
            }
          float s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
          s += __shfl_xor(s, 32, 64);
          res[tb] = MSPair{ga.cap, s};
          if constexpr (kLs) {
            const float z = (z4[0] + z4[1]) + (z4[2] + z4[3]);
            zres[tb] = z + __shfl_xor(z, 32, 64);
          }
          __builtin_amdgcn_sched_barrier(0);
          continue;
        }
        if constexpr (kLs) {
          float z4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int vb = 0; vb < 4; ++vb)
#pragma unroll
            for (int r = 0; r < 16; ++r) z4[r & 3] += (kTail && x[vb][r] == -INFINITY) ? 0.0f : x[vb][r];
          const float z = (z4[0] + z4[1]) + (z4[2] + z4[3]);
          zres[tb] = z + __shfl_xor(z, 32, 64);
        }
        float m4[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (int vb = 0; vb < 4; ++vb)
#pragma unroll
          for (int r = 0; r < 16; ++r) m4[r & 3] = fmaxf(m4[r & 3], x[vb][r]);
        float m = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
        m = fmaxf(m, __shfl_xor(m, 32, 64));
        const float ms = m * kLog2e;
        float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int vb = 0; vb < 4; ++vb)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            s4[r & 3] += __builtin_amdgcn_exp2f(fmaf(x[vb][r], kLog2e, -ms));
        float s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
        s += __shfl_xor(s, 32, 64);
        res[tb] = MSPair{m, s};
        __builtin_amdgcn_sched_barrier(0);  // one token block's values live at a time
      }
    };
    if (kFineMask) {
      epilogue(yes{});
    } else if (lo_w < 128 && hi_w > 0) {
      // vocab % 128 == 0: a half that holds any owned row holds 128
      epilogue(no{});
    } else {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) res[tb] = MSPair{-INFINITY, 0.0f};
    }
    // lanes 0-31 hold the (m, s) of token columns t_first + wt*128 + tb*32 + lane
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const int tok = t_first + wt * 128 + tb * 32 + fr;
      if (lane < 32 && tok >= t_own && tok < n_rows) {
        prow[tok] = res[tb];
        if constexpr (kLs) ga.zsum[(int64_t)(2 * vt + wv) * n_rows + tok] = zres[tb];
      }
    }
  }
  // drain the ring's trailing (unused) loads before the workgroup exits
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
}

// lse / per-token loss from the vocab-tile partials. A 512-thread workgroup
// owns 32 tokens (8192 tokens give 256 workgroups, one per CU). Its 8 waves
// first compute the target logits of 4 tokens each (a wave-wide fp32 dot
// product over d), then 16 groups of 32 threads each fold every 16th partial
// (two per vocab tile) with an online (max, sum) merge (coalesced 256-byte
// reads); the 16 partial states are merged in a fixed order through LDS
// (deterministic).
constexpr int kRowsPerBlock = 32;
constexpr int kRowGroups = 16;

__device__ __forceinline__ MSPair ms_merge(MSPair a, MSPair b) {
  const float m = fmaxf(a.m, b.m);
  if (m == -INFINITY) return {m, 0.0f};
  float s = 0.0f;
  if (a.m != -INFINITY) s += a.s * __builtin_amdgcn_exp2f((a.m - m) * kLog2e);
  if (b.m != -INFINITY) s += b.s * __builtin_amdgcn_exp2f((b.m - m) * kLog2e);
  return {m, s};
}

template <typename T>
__global__ void __launch_bounds__(kRowsPerBlock * kRowGroups)
lmhead_ce_rows_kernel(const T* __restrict__ H, const T* __restrict__ W,
                      const MSPair* __restrict__ part, const int64_t* __restrict__ targets,
                      float* __restrict__ lse, float* __restrict__ losses, int n_rows, int vocab,
                      int d, int64_t ldh, int64_t ldw, int n_vt, int64_t ignore_index, float cap,
                      const float* __restrict__ zsum, float ls) {
  constexpr int kPerWave = kRowsPerBlock / (kRowsPerBlock * kRowGroups / 64);  // tokens per wave
  __shared__ MSPair red[kRowGroups][kRowsPerBlock];
  __shared__ float redz[kRowGroups][kRowsPerBlock];
  __shared__ float tl[kRowsPerBlock];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = blockIdx.x * kRowsPerBlock;
  const int r = threadIdx.x % kRowsPerBlock;
  const int grp = threadIdx.x / kRowsPerBlock;
  const int row = row0 + r;
  const int n_part = 2 * n_vt;

  // With up to kAllPart partials per thread (vocab up to 65,536) all of them
  // are loaded before the target logits' loads: both sets are then in flight
  // at once instead of one round trip after another.
  constexpr int kAllPart = 32;
  const bool all_at_once = n_part <= kAllPart * kRowGroups;
  MSPair pre[kAllPart];
  if (all_at_once && row < n_rows) {
#pragma unroll
    for (int k = 0; k < kAllPart; ++k)
      if (grp + k * kRowGroups < n_part) pre[k] = part[(int64_t)(grp + k * kRowGroups) * n_rows + row];
  }

  // target logits of rows row0 + wave * kPerWave + q
  {
    float acc[kPerWave];
    bool ok[kPerWave];
    const T* hp[kPerWave];
    const T* wp[kPerWave];
#pragma unroll
    for (int q = 0; q < kPerWave; ++q) {
      const int row = row0 + wave * kPerWave + q;
      const int64_t t = row < n_rows ? targets[row] : (int64_t)-1;
      ok[q] = row < n_rows && t >= 0 && t < vocab;
      hp[q] = H + (int64_t)(ok[q] ? row : 0) * ldh;
      wp[q] = W + (ok[q] ? t : 0) * ldw;
      acc[q] = 0.0f;
    }
    // all loads of the first two 16-byte chunks per lane (d <= 1024) are
    // issued before any FMA; longer rows continue in a loop
    const int d8 = d / 8;
    Vec16<T> a0[kPerWave], b0[kPerWave], a1[kPerWave], b1[kPerWave];
#pragma unroll
    for (int q = 0; q < kPerWave; ++q) {
      const int c0 = min(lane, d8 - 1), c1 = min(lane + 64, d8 - 1);
      a0[q] = load16<T>(hp[q] + 8 * c0);
      b0[q] = load16<T>(wp[q] + 8 * c0);
      a1[q] = load16<T>(hp[q] + 8 * c1);
      b1[q] = load16<T>(wp[q] + 8 * c1);
    }
#pragma unroll
    for (int q = 0; q < kPerWave; ++q) {
      if (ok[q] && lane < d8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[q] = fmaf(to_f32(a0[q].e[e]), to_f32(b0[q].e[e]), acc[q]);
      }
      if (ok[q] && lane + 64 < d8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[q] = fmaf(to_f32(a1[q].e[e]), to_f32(b1[q].e[e]), acc[q]);
      }
    }
    for (int c = lane + 128; c < d8; c += 64) {
#pragma unroll
      for (int q = 0; q < kPerWave; ++q) {
        if (!ok[q]) continue;
        const Vec16<T> a = load16<T>(hp[q] + 8 * c);
        const Vec16<T> b = load16<T>(wp[q] + 8 * c);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[q] = fmaf(to_f32(a.e[e]), to_f32(b.e[e]), acc[q]);
      }
    }
#pragma unroll
    for (int q = 0; q < kPerWave; ++q) {
      const float v = wave_sum(acc[q]);
      if (lane == 0) tl[wave * kPerWave + q] = v;
    }
  }

  MSPair st{-INFINITY, 0.0f};
  float zs = 0.0f;  // label smoothing: sum of the (capped) logits, fixed order
  if (row < n_rows && all_at_once) {
    // partials grp, grp + kRowGroups, ... merged in that order
#pragma unroll
    for (int k = 0; k < kAllPart; ++k)
      if (grp + k * kRowGroups < n_part) st = ms_merge(st, pre[k]);
    if (zsum) {
      for (int v = grp; v < n_part; v += kRowGroups) zs += zsum[(int64_t)v * n_rows + row];
    }
  } else if (row < n_rows) {
    // 8 partials in flight per thread, then merged in order
    for (int v0 = grp; v0 < n_part; v0 += 8 * kRowGroups) {
      MSPair buf[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int v = min(v0 + i * kRowGroups, n_part - 1);
        buf[i] = part[(int64_t)v * n_rows + row];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (v0 + i * kRowGroups < n_part) st = ms_merge(st, buf[i]);
      if (zsum) {
        for (int i = 0; i < 8; ++i)
          if (v0 + i * kRowGroups < n_part) zs += zsum[(int64_t)(v0 + i * kRowGroups) * n_rows + row];
      }
    }
  }
  red[grp][r] = st;
  redz[grp][r] = zs;
  __syncthreads();
  if (grp != 0 || row >= n_rows) return;
  for (int g = 1; g < kRowGroups; ++g) {
    st = ms_merge(st, red[g][r]);
    zs += redz[g][r];
  }
  const float l = st.m + fast_log(st.s);
  lse[row] = l;
  const int64_t t = targets[row];
  float loss;
  if (t == ignore_index) loss = 0.0f;
  else if (t < 0 || t >= vocab) loss = NAN;
  else {
    float zt = tl[r];
    if (cap > 0.0f) {
      const Cap cp(cap);
      zt = cap + cp.nc * kLn2 * __builtin_amdgcn_rcpf(cp.q(zt) + 1.0f);  // cap * tanh(zt / cap)
    }
    // label smoothing (kernels/ce_fused.py:251-256): lse - (1 - a) z_t - a mean(z)
    loss = zsum ? l - (1.0f - ls) * zt - ls * zs / (float)vocab : l - zt;
  }
  losses[row] = loss;
}

// mean over non-ignored tokens, fixed summation order (one workgroup).
__global__ void __launch_bounds__(1024)
lmhead_ce_mean_kernel(const float* __restrict__ losses, const int64_t* __restrict__ targets,
                      float* __restrict__ loss_out, int64_t* __restrict__ n_valid_out, int n_rows,
                      int64_t ignore_index) {
  float sum = 0.0f;
  int cnt = 0;
#pragma unroll 8
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

// Target entries of the backward: dz[t, target[t]] = (exp(z_t - lse_t) - (1 - a) - a / vocab) * s_t
// with z_t = hidden[t] . weight[target[t]] as an fp32 dot product (one wave per
// token, as the row kernel computes target logits). Ignored tokens and targets
// outside [0, vocab) keep what the tile kernel wrote (0 and NaN rows).
template <typename T>
__global__ void __launch_bounds__(256)
lmhead_ce_grad_target_kernel(const T* __restrict__ H, const T* __restrict__ W, GradArgs ga,
                             int n_rows, int vocab, int d, int64_t ldh, int64_t ldw) {
  const int lane = threadIdx.x & 63;
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= n_rows) return;  // the whole wave
  const int64_t tg = ga.targets[tok];
  if (tg == ga.ignore_index || tg < 0 || tg >= ga.vocab_total) return;
  const int64_t tl = tg - ga.v0;  // the target's column in this range (W starts at row v0)
  if (tl < 0 || tl >= vocab) return;
  const T* hp = H + (int64_t)tok * ldh;
  const T* wp = W + tl * ldw;
  float acc = 0.0f;
  for (int c = lane; c < d / 8; c += 64) {
    const Vec16<T> a = load16<T>(hp + 8 * c);
    const Vec16<T> b = load16<T>(wp + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf(to_f32(a.e[e]), to_f32(b.e[e]), acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    const float gs = ga.grad_loss[0] / ga.denom[0];
    float g;
    if (ga.cap > 0.0f) {
      const Cap cp(ga.cap);
      const float q = cp.q(acc);
      const float r = __builtin_amdgcn_rcpf(q + 1.0f);
      const float p = __builtin_amdgcn_exp2f(fmaf(cp.nc, r, (ga.cap - ga.lse[tok]) * kLog2e));
      g = (p - (1.0f - ga.ls) - ga.ls / (float)ga.vocab_total) * gs * (4.0f * q * r * r);
    } else {
      const float p = __builtin_amdgcn_exp2f((acc - ga.lse[tok]) * kLog2e);
      g = (p - (1.0f - ga.ls) - ga.ls / (float)ga.vocab_total) * gs;
    }
    static_cast<T*>(ga.dz)[(int64_t)tok * ga.ld_dz + tl] = from_f32<T>(g);
  }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct WsLayout {
  size_t part, losses, zsum, total;
};

WsLayout ws_layout(int64_t n_rows, int64_t vocab) {
  const int64_t n_vt = (vocab + kTV - 1) / kTV;
  WsLayout w;
  w.part = 0;
  w.losses = align256((size_t)2 * n_vt * n_rows * sizeof(MSPair));
  w.zsum = w.losses + align256((size_t)n_rows * 4);
  w.total = w.zsum + align256((size_t)2 * n_vt * n_rows * 4);
  return w;
}

template <typename T, bool kCap, bool kLs>
void launch_tiles_fwd(const T* hp, const T* wp, MSPair* part, int n_rows, int vocab, int d,
                      int64_t ldh, int64_t ldw, int n_vt, int n_tt, const GradArgs& ga, dim3 gd,
                      dim3 bd, hipStream_t s) {
  if (vocab >= kTV && n_rows >= kTT && vocab % 128 == 0)
    lmhead_ce_tile_kernel<T, true, false, false, kCap, kLs><<<gd, bd, 0, s>>>(hp, wp, part, n_rows, vocab, d, ldh, ldw, n_vt, n_tt, ga);
  else if (vocab >= kTV && n_rows >= kTT)
    lmhead_ce_tile_kernel<T, true, true, false, kCap, kLs><<<gd, bd, 0, s>>>(hp, wp, part, n_rows, vocab, d, ldh, ldw, n_vt, n_tt, ga);
  else
    lmhead_ce_tile_kernel<T, false, true, false, kCap, kLs><<<gd, bd, 0, s>>>(hp, wp, part, n_rows, vocab, d, ldh, ldw, n_vt, n_tt, ga);
}

template <typename T>
void launch_lmhead(const void* h, const void* w, const int64_t* targets, float* loss, float* lse,
                   float* losses, int64_t* n_valid, void* ws, int n_rows, int vocab, int d,
                   int64_t ldh, int64_t ldw, int64_t ignore_index, float cap, float ls,
                   hipStream_t s) {
  const int n_vt = (vocab + kTV - 1) / kTV;
  const int n_tt = (n_rows + kTT - 1) / kTT;
  const int grid = min(n_vt * n_tt, cu_count());
  WsLayout L = ws_layout(n_rows, vocab);
  char* base = static_cast<char*>(ws);
  MSPair* part = reinterpret_cast<MSPair*>(base + L.part);
  float* lrow = losses ? losses : reinterpret_cast<float*>(base + L.losses);
  const T* hp = static_cast<const T*>(h);
  const T* wp = static_cast<const T*>(w);
  const dim3 gd(grid), bd(kLThreads);
  GradArgs ga{};
  ga.cap = cap;
  ga.ls = ls;
  ga.vocab_total = vocab;
  ga.zsum = ls > 0.0f ? reinterpret_cast<float*>(base + L.zsum) : nullptr;
  if (cap > 0.0f && ls > 0.0f)
    launch_tiles_fwd<T, true, true>(hp, wp, part, n_rows, vocab, d, ldh, ldw, n_vt, n_tt, ga, gd, bd, s);
  else if (cap > 0.0f)
    launch_tiles_fwd<T, true, false>(hp, wp, part, n_rows, vocab, d, ldh, ldw, n_vt, n_tt, ga, gd, bd, s);
  else if (ls > 0.0f)
    launch_tiles_fwd<T, false, true>(hp, wp, part, n_rows, vocab, d, ldh, ldw, n_vt, n_tt, ga, gd, bd, s);
  else
    launch_tiles_fwd<T, false, false>(hp, wp, part, n_rows, vocab, d, ldh, ldw, n_vt, n_tt, ga, gd, bd, s);
  lmhead_ce_rows_kernel<T><<<dim3((n_rows + kRowsPerBlock - 1) / kRowsPerBlock),
                             dim3(kRowsPerBlock * kRowGroups), 0, s>>>(
      hp, wp, part, targets, lse, lrow, n_rows, vocab, d, ldh, ldw, n_vt, ignore_index, cap, ga.zsum, ls);
  lmhead_ce_mean_kernel<<<dim3(1), dim3(1024), 0, s>>>(lrow, targets, loss, n_valid, n_rows,
                                                      ignore_index);
}

template <typename T, bool kCap>
void launch_tiles_bwd(const T* hp, const T* wp, int n_rows, int vocab, int d, int64_t ldh,
                      int64_t ldw, int n_vt, int n_tt, const GradArgs& ga, bool vec_ok, dim3 gd,
                      dim3 bd, hipStream_t s) {
  if (vocab >= kTV && n_rows >= kTT && vocab % 128 == 0 && vec_ok)
    lmhead_ce_tile_kernel<T, true, false, true, kCap><<<gd, bd, 0, s>>>(hp, wp, nullptr, n_rows, vocab, d, ldh, ldw, n_vt, n_tt, ga);
  else if (vocab >= kTV && n_rows >= kTT)
    lmhead_ce_tile_kernel<T, true, true, true, kCap><<<gd, bd, 0, s>>>(hp, wp, nullptr, n_rows, vocab, d, ldh, ldw, n_vt, n_tt, ga);
  else
    lmhead_ce_tile_kernel<T, false, true, true, kCap><<<gd, bd, 0, s>>>(hp, wp, nullptr, n_rows, vocab, d, ldh, ldw, n_vt, n_tt, ga);
}

template <typename T>
void launch_lmhead_bwd(const void* h, const void* w, const GradArgs& ga, int n_rows, int vocab,
                       int d, int64_t ldh, int64_t ldw, hipStream_t s) {
  const int n_vt = (vocab + kTV - 1) / kTV;
  const int n_tt = (n_rows + kTT - 1) / kTT;
  const int grid = min(n_vt * n_tt, cu_count());
  const T* hp = static_cast<const T*>(h);
  const T* wp = static_cast<const T*>(w);
  const dim3 gd(grid), bd(kLThreads);
  const bool vec_ok = ga.ld_dz % 8 == 0 && aligned16(ga.dz);
  if (ga.cap > 0.0f)
    launch_tiles_bwd<T, true>(hp, wp, n_rows, vocab, d, ldh, ldw, n_vt, n_tt, ga, vec_ok, gd, bd, s);
  else
    launch_tiles_bwd<T, false>(hp, wp, n_rows, vocab, d, ldh, ldw, n_vt, n_tt, ga, vec_ok, gd, bd, s);
  lmhead_ce_grad_target_kernel<T><<<dim3((n_rows + 3) / 4), dim3(256), 0, s>>>(hp, wp, ga, n_rows, vocab, d, ldh, ldw);
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
                                int64_t ignore_index, float softcap, float label_smoothing,
                                int dtype, void* stream) {
  const char* name = "ak_lmhead_ce_fwd";
  if (!(softcap >= 0.0f) || softcap == INFINITY)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: softcap must be finite and >= 0", name);
  if (!(label_smoothing >= 0.0f && label_smoothing <= 1.0f))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: label_smoothing must be in [0, 1]", name);
  if (dtype != AK_DTYPE_BF16 && dtype != AK_DTYPE_F16)
    return ak_set_error(AK_ERR_UNSUPPORTED, "%s: dtype must be bf16 or fp16", name);
  if (n_rows <= 0 || vocab <= 0 || d <= 0)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: bad shape n_rows=%lld vocab=%lld d=%lld", name,
                        (long long)n_rows, (long long)vocab, (long long)d);
  if (d % ak::kKB)
    return ak_set_error(AK_ERR_UNSUPPORTED, "%s: d=%lld must be a multiple of %d", name,
                        (long long)d, ak::kKB);
  if (n_rows > (1 << 30) || vocab > (1 << 30) || d > (1 << 20))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: shape too large", name);
  if (ld_h < d || ld_w < d || ld_h % 8 || ld_w % 8 || ld_h >= (1 << 23) || ld_w >= (1 << 23))
    return ak_set_error(AK_ERR_INVALID_ARG,
                        "%s: row pitches must be >= d, multiples of 8 and < 2^23 elements", name);
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
                                (int)n_rows, (int)vocab, (int)d, ld_h, ld_w, ignore_index, softcap,
                                label_smoothing, s);
  else
    ak::launch_lmhead<ak::f16>(hidden, weight, targets, loss, lse, losses, n_valid, workspace,
                               (int)n_rows, (int)vocab, (int)d, ld_h, ld_w, ignore_index, softcap,
                               label_smoothing, s);
  return ak_check_launch(name);
}

extern "C" int ak_lmhead_ce_bwd_range(const void* hidden, const void* weight,
                                      const int64_t* targets, const float* lse,
                                      const float* grad_loss, const float* denom, void* grad_logits,
                                      int64_t ld_gl, int64_t n_rows, int64_t vocab, int64_t v_begin,
                                      int64_t v_count, int64_t d, int64_t ld_h, int64_t ld_w,
                                      int64_t ignore_index, float softcap, float label_smoothing,
                                      int dtype, void* stream) {
  const char* name = "ak_lmhead_ce_bwd_range";
  if (!(softcap >= 0.0f) || softcap == INFINITY)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: softcap must be finite and >= 0", name);
  if (!(label_smoothing >= 0.0f && label_smoothing <= 1.0f))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: label_smoothing must be in [0, 1]", name);
  if (dtype != AK_DTYPE_BF16 && dtype != AK_DTYPE_F16)
    return ak_set_error(AK_ERR_UNSUPPORTED, "%s: dtype must be bf16 or fp16", name);
  if (n_rows <= 0 || vocab <= 0 || d <= 0)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: bad shape n_rows=%lld vocab=%lld d=%lld", name,
                        (long long)n_rows, (long long)vocab, (long long)d);
  if (v_begin < 0 || v_count <= 0 || v_begin > vocab - v_count)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: vocab range [%lld, %lld + %lld) outside [0, %lld)",
                        name, (long long)v_begin, (long long)v_begin, (long long)v_count,
                        (long long)vocab);
  if (d % ak::kKB)
    return ak_set_error(AK_ERR_UNSUPPORTED, "%s: d=%lld must be a multiple of %d", name,
                        (long long)d, ak::kKB);
  if (n_rows > (1 << 30) || vocab > (1 << 30) || d > (1 << 20))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: shape too large", name);
  if (ld_h < d || ld_w < d || ld_h % 8 || ld_w % 8 || ld_h >= (1 << 23) || ld_w >= (1 << 23))
    return ak_set_error(AK_ERR_INVALID_ARG,
                        "%s: row pitches must be >= d, multiples of 8 and < 2^23 elements", name);
  if (ld_gl < v_count)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: grad_logits pitch must be >= the range's width", name);
  if (!hidden || !weight || !targets || !lse || !grad_loss || !denom || !grad_logits)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  if (!ak::aligned16(hidden) || !ak::aligned16(weight) ||
      (reinterpret_cast<uintptr_t>(grad_logits) & 1u))
    return ak_set_error(AK_ERR_INVALID_ARG,
                        "%s: hidden and weight must be 16-byte aligned, grad_logits element-aligned", name);
  const int64_t n_tiles = ((v_count + ak::kTV - 1) / ak::kTV) * ((n_rows + ak::kTT - 1) / ak::kTT);
  if (n_tiles > 0x7FFFFFFF) return ak_set_error(AK_ERR_INVALID_ARG, "%s: too many tiles", name);
  ak::GradArgs ga{lse, targets, grad_loss, denom, grad_logits, ld_gl, ignore_index, softcap,
                  label_smoothing, nullptr, v_begin, vocab};
  hipStream_t s = ak_stream(stream);
  // the range's weight rows start at v_begin (16-byte aligned: ld_w is a multiple of 8)
  const void* wr = static_cast<const char*>(weight) + (size_t)v_begin * (size_t)ld_w * 2;
  if (dtype == AK_DTYPE_BF16)
    ak::launch_lmhead_bwd<ak::bf16>(hidden, wr, ga, (int)n_rows, (int)v_count, (int)d, ld_h, ld_w, s);
  else
    ak::launch_lmhead_bwd<ak::f16>(hidden, wr, ga, (int)n_rows, (int)v_count, (int)d, ld_h, ld_w, s);
  return ak_check_launch(name);
}

extern "C" int ak_lmhead_ce_bwd(const void* hidden, const void* weight, const int64_t* targets,
                                const float* lse, const float* grad_loss, const float* denom,
                                void* grad_logits, int64_t ld_gl, int64_t n_rows, int64_t vocab,
                                int64_t d, int64_t ld_h, int64_t ld_w, int64_t ignore_index,
                                float softcap, float label_smoothing, int dtype, void* stream) {
  // the whole vocabulary as one range (errors name ak_lmhead_ce_bwd_range)
  return ak_lmhead_ce_bwd_range(hidden, weight, targets, lse, grad_loss, denom, grad_logits, ld_gl,
                                n_rows, vocab, 0, vocab, d, ld_h, ld_w, ignore_index, softcap,
                                label_smoothing, dtype, stream);
}
