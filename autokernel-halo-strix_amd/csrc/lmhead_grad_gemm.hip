// Gradient GEMMs of the lm-head + cross-entropy backward on the gfx950
// matrix cores, from the dlogits that ak_lmhead_ce_bwd_range writes
// (token-major, [n_rows, ld_dl]):
//   grad_hidden[t, :] = sum_v dlogits[t, v] weight[v, :]   (M = tokens, K = vocab)
//   grad_weight[v, :] = sum_t dlogits[t, v] hidden[t, :]   (M = vocab,  K = tokens)
// They replace the two torch.mm calls of the reference's chunked backward
// (kernels/hip/chunked_linear_cross_entropy.py:121-132).
//
// Both products are C[M, N] = A[M, K] B[K, N] with N = d, fp32 accumulation
// (v_mfma_f32_32x32x16_{bf16,f16}). B (weight or hidden) is stored with its
// N dimension contiguous ("MN-major": row k holds B[k, :]); A is dlogits,
// K-major for grad_hidden (row t holds the K = vocab entries) and MN-major
// for grad_weight (row t holds the M = vocab entries). Neither operand is
// transposed in memory: an MN-major operand is staged in LDS as it lies in
// HBM (64 K-rows x 256 MN entries per K block) and its MFMA fragments are
// read with ds_read_b64_tr_b16, the gfx950 transposing LDS read: each
// 16-lane group names 4 consecutive K-rows x 4 eight-byte pieces and every
// lane receives 4 consecutive K values of one MN column. Two such reads
// give a lane the 8 K values a 32x32x16 operand fragment needs.
//
// Mechanics shared with the lm-head forward kernel: one 256-thread
// workgroup per CU (4 waves, each 128 x 128 of a 256 x 256 output tile in
// 256 accumulator registers), K blocks of 64 staged by global_load_lds into a
// 5-slot ring that runs across work items, operands loaded two blocks ahead,
// fragments read two 16-wide K slices ahead, one barrier per K block.
//
// Work split: M x N tiles of 256 x 256; with T tiles, K blocks KB and G
// workgroups, the first R*G tiles (R = T / G full rounds) run whole and
// store C directly; the remaining tiles are cut into S K ranges each
// (S chosen to balance the rounds: at the C4 shape grad_hidden has 96 tiles
// of 786 K blocks and runs 8 ranges each, grad_weight 591 tiles of 128 and
// splits the 79 tiles of its last round 3 ways). A split range writes an
// fp32 partial tile; lmhead_grad_reduce_kernel then sums the S partials of a
// tile in a fixed order (deterministic) into C. Within each round the items
// are dealt so that the 32 workgroups of one XCD take consecutive items
// (N tiles fastest): the N tiles that share an A row block run together and
// read it from that XCD's L2.
//
// Edges: loads go through buffer resources whose extent ends at the last
// valid row, so rows past M (K-major A) and rows past K (MN-major operands)
// load as zeros; columns past M or N are clamped inside the row and not
// stored. A K-major A's columns past K must hold zeros (its row pitch covers
// the K blocks; the host zeroes dlogits' padding columns).
#include "mfma_ring.h"

#include "scan_buffer.h"

namespace ak {
namespace {

constexpr int kGT = 256;           // output tile edge
constexpr int kMnRowBytes = 512;   // one staged MN-major row: 256 entries x 2 bytes

// 16-byte chunk swizzle of a staged MN-major row, by row mod 4. The 16 lanes
// of one transposing read cover rows 4q..4q+3 x 2 chunks, a 32-lane half
// 4 rows x 4 chunks; with these keys both sets land in distinct LDS banks.
__device__ __forceinline__ int mn_swz(int r4) { return (0xAC60 >> (4 * r4)) & 15; }  // 0, 6, 12, 10

// Division by a divisor fixed per launch: q = mulhi(n, magic) with magic =
// floor(2^32 / d) + 1 for d >= 2 (q = n for d = 1, whose magic would need 33
// bits), exact while n * d < 2^32 (the host checks the bound).
struct FastDiv {
  uint32_t d, magic;
};

__host__ __device__ inline FastDiv fast_div(uint32_t d) {
  return FastDiv{d, d > 1 ? (uint32_t)((1ull << 32) / d + 1) : 0u};
}

__device__ __forceinline__ int fdiv(uint32_t n, FastDiv f) {
  return f.d == 1 ? (int)n : (int)__umulhi(n, f.magic);
}

struct GemmArgs {
  const void* a;   // dlogits
  const void* b;   // weight (grad_hidden) or hidden (grad_weight)
  void* c;         // output [M, N] with pitch ldc, element type per out_mode
  float* part;     // fp32 256 x 256 partial tiles of the split items
  int64_t lda, ldb, ldc;
  int a_cols;      // MN-major A: readable entries per row (>= M, multiple of 8)
  int m, n, k;
  int n_tm, n_tn, kb;
  int n_full;      // items [0, n_full) are whole tiles
  int split;       // K ranges per remaining tile
  int n_items;
  int out_mode;    // 0: store T, 1: store fp32, 2: add into fp32
  FastDiv by_tn, by_rest, by_split;  // divisions by n_tn, the split tiles' count, split
};

enum { kOutT = 0, kOutF32 = 1, kOutF32Add = 2 };

// Item w: tile (tm, tn), K blocks [k0, k1), partial slot (-1: direct store).
struct Item {
  int tm, tn, k0, k1, pslot;
};

__device__ __forceinline__ Item item_at(const GemmArgs& g, int w) {
  Item it;
  int t;
  if (w < g.n_full) {
    t = w;
    it.k0 = 0;
    it.k1 = g.kb;
    it.pslot = -1;
  } else {
    const int r = w - g.n_full;
    const int s = fdiv(r, g.by_rest);
    t = g.n_full + (r - s * (int)g.by_rest.d);
    it.k0 = fdiv(s * g.kb, g.by_split);
    it.k1 = fdiv((s + 1) * g.kb, g.by_split);
    it.pslot = r;
  }
  it.tm = fdiv(t, g.by_tn);
  it.tn = t - it.tm * g.n_tn;
  return it;
}

// 16 MFMAs of one K slice with kDs LDS reads and kDmaN DMA loads spread
// over them (one read after each of the first kDs MFMAs, one DMA after each
// of the last kDmaN).
template <int kDs, int kDmaN>
__device__ __forceinline__ void gemm_slice_order() {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (i < kDs) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    if (i >= 16 - kDmaN) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// ds_read_b64_tr_b16 at LDS byte address addr + kOff, as inline assembly:
// with the compiler's builtin for it the compiler waits for every
// outstanding global-to-LDS load (vmcnt(0)) before each read, which drains
// the ring's prefetch. The kernel orders these reads itself: the slots they
// read have been waited for (vmcnt) and published (barrier) before, and
// frags_ready() ties the fragments to an lgkmcnt(0) wait ahead of their MFMAs.
template <int kOff>
__device__ __forceinline__ u32x2 lds_read_tr(uint32_t addr) {
  u32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(kOff));
  return v;
}

template <typename T, bool kAMn>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
lmhead_grad_gemm_kernel(GemmArgs g) {
  __shared__ u32x4 lds[kSlots * kSlotChunks];  // 160 KiB ring
  char* const ldsb = reinterpret_cast<char*>(lds);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wv = wave >> 1;  // M half of the tile
  const int wt = wave & 1;   // N half
  const int G = (int)gridDim.x;
  const int b = (int)blockIdx.x;
  // position within a round: the 32 workgroups of an XCD (b % 8) take
  // consecutive items
  const int lb = (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;
  if (lb >= g.n_items) return;
  const int n_my = (g.n_items - 1 - lb) / G + 1;

  // ---- DMA ----
  // K-major A: instruction j fills rows lrow + 8 j of the slot (8 rows x 128
  // B); lane i fetches the logical chunk the swizzle (row / 2 mod 8) puts at
  // physical chunk i % 8.
  const int lrow = wave * 64 + (lane >> 3);
  const uint32_t c16[2] = {16u * (uint32_t)((lane & 7) ^ (lane >> 4)),
                           16u * (uint32_t)((lane & 7) ^ ((lane >> 4) + 4))};
  // MN-major operands: instruction j fills rows 16 wave + 2 j + (lane / 32)
  // (two 512-byte rows); lane i takes physical chunk i % 32 of its row.
  const int mrow = 16 * wave + (lane >> 5);  // + 2 j
  const int pchunk = lane & 31;
  const int swz[2] = {mn_swz((lane >> 5) & 3), mn_swz(((lane >> 5) + 2) & 3)};  // by j parity

  // Load state of one operand over this workgroup's sequence of (item, K
  // block). Everything but the per-lane offsets vo is wave-uniform (the item
  // fields pass through readfirstlane, so that the per-block address
  // arithmetic stays scalar); vo depends on the item only.
  struct Op {
    int it, blk, nblk, k0;
    int mn0;             // first M (A) or N (B) index of the item's tile
    const char* slab0;   // the item's K block 0
    uint32_t vo[2];      // per lane, by instruction parity
  };
  const uint32_t lda_b = (uint32_t)g.lda * 2u, ldb_b = (uint32_t)g.ldb * 2u;
  auto op_item = [&](Op& o, bool is_a) {
    const Item x = item_at(g, min(o.it, n_my - 1) * G + lb);
    o.k0 = __builtin_amdgcn_readfirstlane(x.k0);
    o.nblk = __builtin_amdgcn_readfirstlane(x.k1) - o.k0;
    o.mn0 = __builtin_amdgcn_readfirstlane(is_a ? x.tm : x.tn) * kGT;
    if (is_a && !kAMn) {
      o.slab0 = static_cast<const char*>(g.a) + (int64_t)o.mn0 * g.lda * 2;
      o.vo[0] = (uint32_t)lrow * lda_b + c16[0];
      o.vo[1] = (uint32_t)lrow * lda_b + c16[1];
    } else {
      const int cols = is_a ? g.a_cols : g.n;
      const uint32_t ld_b = is_a ? lda_b : ldb_b;
      o.slab0 = static_cast<const char*>(is_a ? g.a : g.b);
#pragma unroll
      for (int jp = 0; jp < 2; ++jp)
        o.vo[jp] = (uint32_t)mrow * ld_b + 2u * (uint32_t)min(o.mn0 + 8 * (pchunk ^ swz[jp]), cols - 8);
    }
  };
  auto op_next = [&](Op& o, bool is_a) {
    if (++o.blk == o.nblk) {
      o.blk = 0;
      ++o.it;
      op_item(o, is_a);
    }
  };
  // Loads go through buffer resources over the valid part of the block:
  // a row past M (K-major A) or past K (MN-major operands) lies beyond the
  // resource's extent and loads zeros into LDS (hardware range check on
  // the per-lane offset), so no block needs a branch. Per instruction the
  // lane offset is the item's vo plus the instruction's row step.
  // MN-major operand rows [64 kbi, 64 kbi + 64) into `slot`
  auto mn_dma = [&](const Op& o, uint32_t ld_b, int slot, int kbi, int j0, int j1) {
    const int rows = min(g.k - kbi * kKB, kKB);
    const Rsrc r = make_rsrc(o.slab0 + (int64_t)kbi * kKB * (int64_t)ld_b, (uint32_t)rows * ld_b);
    char* dst = ldsb + slot * (kSlotChunks * 16) + 16 * wave * kMnRowBytes;
#pragma unroll
    for (int j = j0; j < j1; ++j) bdma16(r, o.vo[j & 1] + (uint32_t)(2 * j) * ld_b, dst + 2 * j * kMnRowBytes);
  };
  // A of (item, block) into `slot`, instructions [j0, j1)
  auto dma_a = [&](const Op& o, int slot, int j0, int j1) {
    const int kbi = o.k0 + o.blk;
    if constexpr (!kAMn) {
      const int rows = min(g.m - o.mn0, kGT);
      const Rsrc r = make_rsrc(o.slab0 + (int64_t)kbi * (kKB * 2), (uint32_t)(rows - 1) * lda_b + kKB * 2);
      u32x4* blk = lds + slot * kSlotChunks + wave * 64 * kChunks;
#pragma unroll
      for (int j = j0; j < j1; ++j) bdma16(r, o.vo[j & 1] + (uint32_t)(8 * j) * lda_b, blk + 8 * j * kChunks);
    } else {
      mn_dma(o, lda_b, slot, kbi, j0, j1);
    }
  };
  auto dma_b = [&](const Op& o, int slot, int j0, int j1) { mn_dma(o, ldb_b, slot, o.k0 + o.blk, j0, j1); };

  // ---- fragment reads ----
  // K-major A: rows wv*128 + 32 i + lane % 32, chunk (2 kk + lane / 32)
  // under the (row / 2 mod 8) swizzle, one ds_read_b128.
  const int fr = lane & 31;
  const int fsw = (fr >> 1) & 7;
  const int khalf = lane >> 5;
  const int arow = (wv * 128 + fr) * kChunks;
  // MN-major: 16-lane group q = lane / 16 reads K-rows 16 kk + 8 (q / 2) +
  // (lane % 16) / 4 (+ 4 for the fragment's upper half) at MN columns
  // 32 i + 16 (q % 2) + 4 (lane % 4) of the wave's 128-column half.
  const int tq = lane >> 4, tj = lane & 15;
  const int tr_row = 8 * (tq >> 1) + (tj >> 2);
  auto tr_off = [&](int half, int i) {
    const int c = ((4 * i + 2 * (tq & 1) + ((tj & 3) >> 1)) ^ mn_swz(tj >> 2)) + 16 * half;
    return tr_row * kMnRowBytes + 16 * c + 8 * (tj & 1);
  };
  int a_off[4], b_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a_off[i] = tr_off(wv, i);
    b_off[i] = tr_off(wt, i);
  }
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)ldsb);
  auto frag_tr = [&](int slot, int off, auto kk_tag) {
    constexpr int kOff = decltype(kk_tag)::value * 16 * kMnRowBytes;
    const uint32_t a = lds0 + (uint32_t)(slot * (kSlotChunks * 16) + off);
    const u32x2 lo = lds_read_tr<kOff>(a);
    const u32x2 hi = lds_read_tr<kOff + 4 * kMnRowBytes>(a);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };
  auto load_frags = [&](int sa, int sb, auto kk_tag, u32x4* a, u32x4* bq) {
    constexpr int kk = decltype(kk_tag)::value;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (kAMn) a[i] = frag_tr(sa, a_off[i], kk_tag);
      else a[i] = lds[sa * kSlotChunks + arow + 32 * i * kChunks + ((2 * kk + khalf) ^ fsw)];
      bq[i] = frag_tr(sb, b_off[i], kk_tag);
    }
  };
  // The transposing reads of a slice's fragments have completed: a wait the
  // fragments pass through, so that no MFMA reading them is scheduled ahead
  // of it.
  auto frags_ready = [&](u32x4* a, u32x4* bq) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(bq[0]), "+v"(bq[1]),
                   "+v"(bq[2]), "+v"(bq[3]));
  };

  f32x16_t acc[4][4];
  u32x4 af[4][4], bf[4][4];  // fragments of the 4 slices of a K block
  auto mfmas = [&](auto first_tag, const u32x4* a, const u32x4* bq) {
    constexpr bool kFirst = decltype(first_tag)::value;
#pragma unroll
    for (int vb = 0; vb < 4; ++vb)
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
        acc[vb][tb] = mfma32(T(), a[vb], bq[tb], kFirst ? f32x16_t{} : acc[vb][tb]);
  };
  constexpr int kReads = kAMn ? 0 : 4;  // compiler-visible LDS reads per slice (the b128 ones)

  // ---- prologue: operand blocks q = 0..3 (A0 B0 A1 B1), block q in slot q % 5 ----
  Op ca{}, cb{};
  op_item(ca, true);
  op_item(cb, false);
  dma_a(ca, 0, 0, kDma);
  op_next(ca, true);
  dma_b(cb, 1, 0, kDma);
  op_next(cb, false);
  dma_a(ca, 2, 0, kDma);
  dma_b(cb, 3, 0, kDma);
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(2 * kDma));  // q = 0, 1 landed
  ring_barrier();

  // Slots of K block j (counted over all of this workgroup's blocks): A in
  // (2j) % 5, B in (2j + 1) % 5. Block j loads A of block j + 2 into slot
  // (2j + 4) % 5 during slices 0-1; after the barrier (every wave is done
  // with block j's slots, block j + 1's slots have landed) B of block j + 2
  // goes into block j's A slot during slices 2-3.
  int sa = 0, sb = 1;
  auto block = [&](auto first_tag, auto last_tag) {
    constexpr bool kLastBlk = decltype(last_tag)::value;
    op_next(ca, true);
    op_next(cb, false);
    const int pa = sa + 4 >= kSlots ? sa + 4 - kSlots : sa + 4;
    const int nsa = sa + 2 >= kSlots ? sa + 2 - kSlots : sa + 2;
    const int nsb = sb + 2 >= kSlots ? sb + 2 - kSlots : sb + 2;
    // each slice first waits for its own fragments (read two slices
    // earlier), then reads those of the slice after next
    frags_ready(af[0], bf[0]);
    load_frags(sa, sb, std::integral_constant<int, 2>{}, af[2], bf[2]);
    mfmas(first_tag, af[0], bf[0]);
    dma_a(ca, pa, 0, kDma / 2);
    gemm_slice_order<kReads, kDma / 2>();
    frags_ready(af[1], bf[1]);
    load_frags(sa, sb, std::integral_constant<int, 3>{}, af[3], bf[3]);
    mfmas(std::false_type{}, af[1], bf[1]);
    dma_a(ca, pa, kDma / 2, kDma);
    gemm_slice_order<kReads, kDma / 2>();
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(kDma));
    ring_barrier();
    frags_ready(af[2], bf[2]);
    if (!kLastBlk) load_frags(nsa, nsb, std::integral_constant<int, 0>{}, af[0], bf[0]);
    mfmas(std::false_type{}, af[2], bf[2]);
    dma_b(cb, sa, 0, kDma / 2);
    if constexpr (kLastBlk) gemm_slice_order<0, kDma / 2>();
    else gemm_slice_order<kReads, kDma / 2>();
    frags_ready(af[3], bf[3]);
    if (!kLastBlk) load_frags(nsa, nsb, std::integral_constant<int, 1>{}, af[1], bf[1]);
    mfmas(std::false_type{}, af[3], bf[3]);
    dma_b(cb, sa, kDma / 2, kDma);
    if constexpr (kLastBlk) gemm_slice_order<0, kDma / 2>();
    else gemm_slice_order<kReads, kDma / 2>();
    sa = nsa;
    sb = nsb;
  };

  using yes = std::true_type;
  using no = std::false_type;
  for (int it = 0; it < n_my; ++it) {
    Item x = item_at(g, it * G + lb);
    x.tm = __builtin_amdgcn_readfirstlane(x.tm);
    x.tn = __builtin_amdgcn_readfirstlane(x.tn);
    x.pslot = __builtin_amdgcn_readfirstlane(x.pslot);
    const int nb = __builtin_amdgcn_readfirstlane(x.k1) - __builtin_amdgcn_readfirstlane(x.k0);
    load_frags(sa, sb, std::integral_constant<int, 0>{}, af[0], bf[0]);
    load_frags(sa, sb, std::integral_constant<int, 1>{}, af[1], bf[1]);
    if (nb == 1) {
      block(yes{}, yes{});
    } else {
      block(yes{}, no{});
      for (int kb = 1; kb < nb - 1; ++kb) block(no{}, no{});
      block(no{}, yes{});
    }
    // the epilogue reads the accumulators with v_accvgpr_read: give the
    // last MFMAs that wrote them (16 passes at most) their wait states
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");

    // ---- epilogue ----
    // accumulator r of block (vb, tb) is C[m0 + wv*128 + 32 vb + 8 (r / 4)
    // + 4 (lane / 32) + r % 4][n0 + wt*128 + 32 tb + lane % 32]
    const int m0 = x.tm * kGT, n0 = x.tn * kGT;
    const int ml = wv * 128 + 4 * khalf;  // + 32 vb + 8 (r / 4) + r % 4
    const int nl = wt * 128 + fr;         // + 32 tb
    if (x.pslot >= 0) {
      float* pt = g.part + (int64_t)x.pslot * (kGT * kGT) + ml * kGT + nl;
#pragma unroll
      for (int vb = 0; vb < 4; ++vb)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          float* q = pt + 32 * vb * kGT + 32 * tb;
#pragma unroll
          for (int r = 0; r < 16; ++r) q[(8 * (r >> 2) + (r & 3)) * kGT] = acc_read(acc[vb][tb][r]);
          __builtin_amdgcn_sched_barrier(0);  // one block's addresses live at a time
        }
    } else {
#pragma unroll
      for (int vb = 0; vb < 4; ++vb)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          const int n = n0 + nl + 32 * tb;
          const int mb = m0 + ml + 32 * vb;
          const int64_t o = (int64_t)mb * g.ldc + n;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int dm = 8 * (r >> 2) + (r & 3);
            const float v = acc_read(acc[vb][tb][r]);
            if (mb + dm < g.m && n < g.n) {
              const int64_t oo = o + (int64_t)dm * g.ldc;
              if (g.out_mode == kOutT) static_cast<T*>(g.c)[oo] = from_f32<T>(v);
              else if (g.out_mode == kOutF32) static_cast<float*>(g.c)[oo] = v;
              else static_cast<float*>(g.c)[oo] += v;
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
    }
  }
  // drain the ring's trailing (unused) loads before the workgroup exits
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
}

// Sum of the S partial tiles of each split tile, in the order of their K
// ranges, into C. Grid (rest tiles, 64) x 256 threads: one float4 of the
// 256 x 256 tile per thread.
template <typename T>
__global__ void __launch_bounds__(256) lmhead_grad_reduce_kernel(GemmArgs g) {
  const int rest = g.n_tm * g.n_tn - g.n_full;
  const int ti = blockIdx.x;  // split tile index (partial slot of range 0)
  const int q = blockIdx.y * 256 + threadIdx.x;
  const int row = q >> 6, col = 4 * (q & 63);
  const int t = g.n_full + ti;
  const int m = (t / g.n_tn) * kGT + row;
  const int n = (t % g.n_tn) * kGT + col;
  if (m >= g.m || n >= g.n) return;  // n < N implies n + 3 < N (N % 8 == 0)
  const float4* p = reinterpret_cast<const float4*>(g.part) + (int64_t)ti * (kGT * kGT / 4) + q;
  float4 s = p[0];
  for (int k = 1; k < g.split; ++k) {
    const float4 v = p[(int64_t)k * rest * (kGT * kGT / 4)];
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  const int64_t o = (int64_t)m * g.ldc + n;
  if (g.out_mode == kOutT) {
    T* c = static_cast<T*>(g.c) + o;
    c[0] = from_f32<T>(s.x);
    c[1] = from_f32<T>(s.y);
    c[2] = from_f32<T>(s.z);
    c[3] = from_f32<T>(s.w);
  } else {
    float* c = static_cast<float*>(g.c) + o;
    if (g.out_mode == kOutF32Add) {
      c[0] += s.x;
      c[1] += s.y;
      c[2] += s.z;
      c[3] += s.w;
    } else {
      c[0] = s.x;
      c[1] = s.y;
      c[2] = s.z;
      c[3] = s.w;
    }
  }
}

// Tiles, K blocks and the split of the last round's tiles (see the file
// comment). The cost of a split S is the busiest workgroup's K blocks (about
// 1 us each: 256 x 256 x 64 MFMA work per CU) plus the reduce pass, which
// reads the rest x S partial tiles of 256 KiB once (at about 6 TB/s: 0.044
// blocks per tile); ties go to fewer ranges.
GemmArgs plan_gemm(int m, int n, int k, int cus) {
  GemmArgs g{};
  g.m = m;
  g.n = n;
  g.k = k;
  g.n_tm = (m + kGT - 1) / kGT;
  g.n_tn = (n + kGT - 1) / kGT;
  g.kb = (k + kKB - 1) / kKB;
  const int tiles = g.n_tm * g.n_tn;
  const int G = max(1, cus);
  const int R = tiles / G, rest = tiles - R * G;
  int best_s = 1;
  double best = (double)R * g.kb + (rest ? g.kb : 0);
  for (int s = 2; rest && s <= min(16, g.kb); ++s) {
    const double cost = (double)R * g.kb + (double)((rest * s + G - 1) / G) * ((g.kb + s - 1) / s) +
                        0.044 * rest * s;
    if (cost < best) {
      best = cost;
      best_s = s;
    }
  }
  g.split = best_s;
  g.n_full = best_s == 1 ? tiles : R * G;
  g.n_items = g.n_full + (tiles - g.n_full) * best_s;
  g.by_tn = fast_div((uint32_t)g.n_tn);
  g.by_rest = fast_div((uint32_t)max(1, tiles - g.n_full));
  g.by_split = fast_div((uint32_t)g.split);
  return g;
}

// The exactness bound of the launch's divisions (numerator x divisor < 2^32).
bool plan_divisions_exact(const GemmArgs& g) {
  const uint64_t lim = 1ull << 32;
  const int tiles = g.n_tm * g.n_tn;
  return (uint64_t)tiles * g.n_tn < lim && (uint64_t)g.n_items * g.by_rest.d < lim &&
         (uint64_t)(g.split + 1) * g.kb * g.split < lim;
}

size_t part_bytes(const GemmArgs& g) {
  const int rest = g.n_tm * g.n_tn - g.n_full;
  return g.split > 1 ? (size_t)rest * g.split * kGT * kGT * sizeof(float) : 0;
}

template <typename T>
void launch_gemm(const GemmArgs& g, bool a_mn, hipStream_t s) {
  const int grid = min(g.n_items, cu_count());
  if (a_mn) lmhead_grad_gemm_kernel<T, true><<<dim3(grid), dim3(256), 0, s>>>(g);
  else lmhead_grad_gemm_kernel<T, false><<<dim3(grid), dim3(256), 0, s>>>(g);
  const int rest = g.n_tm * g.n_tn - g.n_full;
  if (g.split > 1 && rest > 0)
    lmhead_grad_reduce_kernel<T><<<dim3(rest, kGT * kGT / 4 / 256), dim3(256), 0, s>>>(g);
}

// Shared argument checks; fills the problem-independent fields of *g.
int check_gemm(const char* name, int64_t n_rows, int64_t vocab, int64_t d, const void* dl,
               int64_t ld_dl, const void* b, int64_t ldb, const void* c, int64_t ldc,
               int out_mode, int dtype) {
  if (dtype != AK_DTYPE_BF16 && dtype != AK_DTYPE_F16)
    return ak_set_error(AK_ERR_UNSUPPORTED, "%s: dtype must be bf16 or fp16", name);
  if (out_mode < kOutT || out_mode > kOutF32Add)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: out_mode must be 0 (input dtype), 1 (fp32) or 2 (fp32 add)", name);
  if (n_rows <= 0 || vocab <= 0 || d <= 0)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: bad shape n_rows=%lld vocab=%lld d=%lld", name,
                        (long long)n_rows, (long long)vocab, (long long)d);
  if (d % kKB)
    return ak_set_error(AK_ERR_UNSUPPORTED, "%s: d=%lld must be a multiple of %d", name, (long long)d, kKB);
  if (n_rows > (1 << 30) || vocab > (1 << 30) || d > (1 << 20))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: shape too large", name);
  // the launch plan counts tiles, and up to 16 K ranges of each, in int
  const int64_t m_tiles = (std::max(n_rows, vocab) + kGT - 1) / kGT, n_tiles = (d + kGT - 1) / kGT;
  if (m_tiles * n_tiles * 16 >= (int64_t(1) << 31))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: too many 256 x 256 output tiles", name);
  const int64_t vpad = (vocab + kKB - 1) / kKB * kKB;
  if (ld_dl < vpad || ld_dl % 8 || ld_dl >= (1 << 23))
    return ak_set_error(AK_ERR_INVALID_ARG,
                        "%s: dlogits pitch must cover vocab rounded up to %d (zero padding), be a "
                        "multiple of 8 and < 2^23 elements", name, kKB);
  if (ldb < d || ldb % 8 || ldb >= (1 << 23))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: operand pitch must be >= d, a multiple of 8 and < 2^23", name);
  if (ldc < d) return ak_set_error(AK_ERR_INVALID_ARG, "%s: output pitch must be >= d", name);
  if (!dl || !b || !c) return ak_set_error(AK_ERR_INVALID_ARG, "%s: null pointer", name);
  if (!aligned16(dl) || !aligned16(b))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: dlogits and the operand must be 16-byte aligned", name);
  const size_t esz = out_mode == kOutT ? 2 : 4;
  if (reinterpret_cast<uintptr_t>(c) % esz)
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: output not element-aligned", name);
  return AK_OK;
}

int run_gemm(const char* name, GemmArgs g, bool a_mn, void* ws, size_t ws_bytes, int dtype,
             hipStream_t s) {
  if (!plan_divisions_exact(g))
    return ak_set_error(AK_ERR_INVALID_ARG, "%s: problem too large for the tile schedule", name);
  const size_t need = part_bytes(g);
  if (need && (!ws || ws_bytes < need))
    return ak_set_error(AK_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu", name, ws_bytes, need);
  if (need && !aligned16(ws)) return ak_set_error(AK_ERR_INVALID_ARG, "%s: workspace not 16-byte aligned", name);
  g.part = static_cast<float*>(ws);
  if (dtype == AK_DTYPE_BF16) launch_gemm<bf16>(g, a_mn, s);
  else launch_gemm<f16>(g, a_mn, s);
  return ak_check_launch(name);
}

}  // namespace
}  // namespace ak

extern "C" size_t ak_lmhead_grad_workspace_bytes(int64_t n_rows, int64_t vocab, int64_t d) {
  if (n_rows <= 0 || vocab <= 0 || d <= 0 || n_rows > (1 << 30) || vocab > (1 << 30) || d > (1 << 20))
    return 0;
  const int cus = ak::cu_count();
  const size_t h = ak::part_bytes(ak::plan_gemm((int)n_rows, (int)d, (int)vocab, cus));
  const size_t w = ak::part_bytes(ak::plan_gemm((int)vocab, (int)d, (int)n_rows, cus));
  return h > w ? h : w;
}

extern "C" int ak_lmhead_grad_hidden(const void* grad_logits, int64_t ld_gl, const void* weight,
                                     int64_t ld_w, void* grad_hidden, int64_t ld_gh,
                                     int64_t n_rows, int64_t vocab, int64_t d, int out_mode,
                                     void* workspace, size_t workspace_bytes, int dtype,
                                     void* stream) {
  const char* name = "ak_lmhead_grad_hidden";
  int rc = ak::check_gemm(name, n_rows, vocab, d, grad_logits, ld_gl, weight, ld_w, grad_hidden,
                          ld_gh, out_mode, dtype);
  if (rc) return rc;
  ak::GemmArgs g = ak::plan_gemm((int)n_rows, (int)d, (int)vocab, ak::cu_count());
  g.a = grad_logits;
  g.lda = ld_gl;
  g.a_cols = (int)ld_gl;
  g.b = weight;
  g.ldb = ld_w;
  g.c = grad_hidden;
  g.ldc = ld_gh;
  g.out_mode = out_mode;
  return ak::run_gemm(name, g, false, workspace, workspace_bytes, dtype, ak_stream(stream));
}

extern "C" int ak_lmhead_grad_weight(const void* grad_logits, int64_t ld_gl, const void* hidden,
                                     int64_t ld_h, void* grad_weight, int64_t ld_gw,
                                     int64_t n_rows, int64_t vocab, int64_t d, int out_mode,
                                     void* workspace, size_t workspace_bytes, int dtype,
                                     void* stream) {
  const char* name = "ak_lmhead_grad_weight";
  int rc = ak::check_gemm(name, n_rows, vocab, d, grad_logits, ld_gl, hidden, ld_h, grad_weight,
                          ld_gw, out_mode, dtype);
  if (rc) return rc;
  ak::GemmArgs g = ak::plan_gemm((int)vocab, (int)d, (int)n_rows, ak::cu_count());
  g.a = grad_logits;
  g.lda = ld_gl;
  g.a_cols = (int)ld_gl;
  g.b = hidden;
  g.ldb = ld_h;
  g.c = grad_weight;
  g.ldc = ld_gw;
  g.out_mode = out_mode;
  return ak::run_gemm(name, g, true, workspace, workspace_bytes, dtype, ak_stream(stream));
}
