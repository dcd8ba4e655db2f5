/*
 * autokernel_mi355x.h -- C ABI of the gfx950 (MI355X / CDNA4) kernel library
 * libautokernel_gfx950.so.
 *
 * Every entry point:
 *   - takes plain device pointers, element counts and element strides (row
 *     pitches in ELEMENTS, not bytes) plus an opaque HIP stream (hipStream_t
 *     passed as void*, NULL = the null stream);
 *   - enqueues its kernels on that stream and returns without synchronising;
 *   - never allocates or frees device memory (the caller owns every output
 *     and workspace buffer);
 *   - returns AK_OK (0) or a negative AK_ERR_* code; the message for the last
 *     failure on the calling thread is returned by ak_last_error().
 *
 * Float element types are selected by an AK_DTYPE_* code. All reductions are
 * carried in fp32 whatever the storage type.
 *
 * Each declaration names the reference interface (joelhenwang/autokernel-
 * halo-strix, file:line) whose behaviour it replaces.
 */
#ifndef AUTOKERNEL_MI355X_H
#define AUTOKERNEL_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AK_ABI_VERSION 2

#define AK_DTYPE_F32 0
#define AK_DTYPE_F16 1
#define AK_DTYPE_BF16 2
/* complex64 (interleaved fp32 re, im): the selective scan's complex A */
#define AK_DTYPE_C64 3

/* Selective-scan bc_flags: B / C input-independent, [dim, dstate] fp32
 * (complex64 with a complex A) */
#define AK_SCAN_B_CONST 1
#define AK_SCAN_C_CONST 2
/* ak_selective_scan_bwd_workspace_bytes only: the size for a complex A */
#define AK_SCAN_A_COMPLEX 4

#define AK_OK 0
#define AK_ERR_INVALID_ARG (-1)
#define AK_ERR_UNSUPPORTED (-2)
#define AK_ERR_LAUNCH (-3)
#define AK_ERR_WORKSPACE (-4)

/* Message describing the last non-zero return on the calling thread. */
const char* ak_last_error(void);

/* AK_ABI_VERSION of the loaded library. */
int ak_abi_version(void);

/* Name of the GPU architecture the library was built for ("gfx950"). */
const char* ak_target_arch(void);

/*
 * RMSNorm: y[r, :] = (x[r, :] / sqrt(mean(x[r, :]^2) + eps)) * weight.
 * Replaces kernels/hip/rmsnorm.py:119-143 (rmsnorm_hip) and the PyTorch
 * fallback of kernels/hip/rmsnorm.py:156-177 (kernel_fn); semantics of
 * reference.py:25-29 (rmsnorm_ref), computed in fp32 and rounded once.
 */
int ak_rmsnorm_fwd(const void* x, const void* weight, void* y,
                   int64_t rows, int64_t cols, int64_t ld_x, int64_t ld_y,
                   float eps, int dtype, void* stream);

/*
 * Fused residual add + RMSNorm:
 *   h = round_dtype(x + residual)            (written to new_residual if non-NULL)
 *   y = round_dtype((h / sqrt(mean(h^2) + eps)) * weight)
 * Replaces kernels/hip/fused_residual_add_rmsnorm.py:135-169
 * (fused_residual_add_rmsnorm_hip) and :284-319 (..._dual_hip); semantics of
 * reference.py:71-78 (fused_residual_add_rmsnorm_ref).
 */
int ak_fused_add_rmsnorm_fwd(const void* x, const void* residual, const void* weight,
                             void* new_residual, void* y,
                             int64_t rows, int64_t cols,
                             int64_t ld_x, int64_t ld_r, int64_t ld_nr, int64_t ld_y,
                             float eps, int dtype, void* stream);

/*
 * RMSNorm backward, per row in fp32 (x the forward input):
 *   r = 1 / sqrt(mean(x^2) + eps),  n = x * r,  g = grad_out * weight
 *   grad_x      = round_dtype(r * (g - n * sum(g * n) / cols))
 *   grad_weight = sum over rows of grad_out * n           (fp32, [cols])
 * Replaces kernels/hip/rmsnorm_backward.py:239-281 (kernel_fn) and its
 * kernel :60-189 (which accumulated grad_weight with fp32 atomics); the
 * row sums of grad_weight here run in a fixed order (deterministic).
 * grad_weight may be NULL (then no workspace is needed); otherwise workspace
 * must hold ak_rmsnorm_bwd_workspace_bytes(rows, cols) bytes, 16-byte
 * aligned. x, weight, grad_out and grad_x share the element type dtype.
 */
size_t ak_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols);
int ak_rmsnorm_bwd(const void* x, const void* weight, const void* grad_out,
                   void* grad_x, float* grad_weight,
                   void* workspace, size_t workspace_bytes,
                   int64_t rows, int64_t cols,
                   int64_t ld_x, int64_t ld_g, int64_t ld_gx,
                   float eps, int dtype, void* stream);

/*
 * Fused residual add + RMSNorm backward: the RMSNorm backward above applied
 * to the saved hidden state (x + residual) and grad_normed, plus grad_hidden:
 *   grad_x = grad_residual = round_dtype(grad_hidden + r * (g - n * sum(g * n) / cols))
 * with g = grad_normed * weight; grad_hidden may be NULL (treated as zero).
 * Replaces kernels/hip/fused_residual_rmsnorm_backward.py:248-298
 * (kernel_fn) and its kernel :61-197. Workspace as for ak_rmsnorm_bwd.
 */
int ak_fused_add_rmsnorm_bwd(const void* hidden, const void* weight,
                             const void* grad_hidden, const void* grad_normed,
                             void* grad_x, float* grad_weight,
                             void* workspace, size_t workspace_bytes,
                             int64_t rows, int64_t cols,
                             int64_t ld_h, int64_t ld_gh, int64_t ld_gn, int64_t ld_gx,
                             float eps, int dtype, void* stream);

/*
 * ak_fused_add_rmsnorm_bwd without a workspace: the same kernels and results
 * (bitwise), with the partial weight-gradient rows in a fixed 64 MiB device
 * array inside the library (one per GPU, held until the process ends) instead
 * of a caller buffer. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * or training loops, harnesses that forbid hipMalloc); it calls no hipMalloc,
 * hipFree or allocating routine. grad_hidden = NULL gives the plain RMSNorm
 * backward of ak_rmsnorm_bwd (x passed as hidden). Shapes whose partial rows
 * (at most 256 workgroup slots, 1024 for rows of <= 512 bf16 / fp16 elements)
 * times cols x 4 bytes exceed 16 MiB -- cols > 16384 for a full grid -- are
 * rejected with AK_ERR_WORKSPACE; use ak_fused_add_rmsnorm_bwd for those. The
 * array holds four 16 MiB slots per GPU; each stream that calls this on a
 * device gets a slot of its own on its first call (for the life of the
 * process), so calls queued on different streams -- a captured graph
 * replayed beside eager calls, say -- never share partial rows, and calls on
 * one stream are ordered by it. A fifth stream on one device is refused with
 * AK_ERR_UNSUPPORTED. A slot keeps its last call's contents. A graph captured
 * on one stream and replayed on another keeps the capture stream's slot, so it
 * must not overlap eager calls on the capture stream. The per-thread default
 * stream counts as one stream. The first call on each device looks up the
 * array's address on it.
 */
int ak_fused_add_rmsnorm_bwd_noalloc(const void* hidden, const void* weight,
                                     const void* grad_hidden, const void* grad_normed,
                                     void* grad_x, float* grad_weight,
                                     int64_t rows, int64_t cols,
                                     int64_t ld_h, int64_t ld_gh, int64_t ld_gn, int64_t ld_gx,
                                     float eps, int dtype, void* stream);

/*
 * Row softmax over the last dimension with fp32 accumulation.
 * Replaces kernels/hip/softmax.py:273-326 (softmax_hip); semantics of
 * reference.py:14-17 (softmax_ref). -inf entries give exact zeros.
 */
int ak_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols,
                   int64_t ld_x, int64_t ld_y, int dtype, void* stream);

/*
 * Cross-entropy forward over materialised logits [rows, vocab].
 * Replaces kernels/ce_fused.py:333-382 (cross_entropy_fwd_hip).
 * Writes per-row loss and logsumexp; row_max / row_sum when non-NULL
 * (tiny mode); grad_logits (same dtype as logits) when non-NULL (fused mode),
 * pre-multiplied by scale_grad and, when scale_dev is non-NULL, by the
 * device value scale_dev[0] (e.g. 1 / #counted rows from ak_ce_count_valid,
 * so the mean's scale needs no host read); z_loss_weight w >= 0 adds the
 * gradient of w * lse^2 to it (as in ak_ce_bwd_tiny). softcap <= 0 disables the logit
 * softcap, label_smoothing <= 0 disables smoothing. Rows whose target equals
 * ignore_index get loss 0 and a zero gradient row; a target outside
 * [0, vocab) that is not ignore_index yields loss NaN. Rows are walked by
 * grid stride: any row count whose extent fits 64-bit addressing.
 */
int ak_ce_fwd(const void* logits, const int64_t* targets,
              float* losses, float* lse, float* row_max, float* row_sum,
              void* grad_logits,
              int64_t rows, int64_t vocab, int64_t ld_logits, int64_t ld_grad,
              float softcap, int64_t ignore_index, float label_smoothing,
              float scale_grad, float z_loss_weight, const float* scale_dev,
              int dtype, void* stream);

/*
 * Cross-entropy backward from saved row max / row sum (tiny mode):
 *   grad[r, i] = (p_ri (1 + 2 w lse_r) - [i == t_r](1 - a) - a / vocab)
 *                * (softcap > 0 ? 1 - tanh^2(logit / softcap) : 1) * scale
 * with p and lse over the (capped) logits, w = z_loss_weight (the gradient
 * of w * lse^2, the z-loss the reference added in PyTorch,
 * kernels/ce_fused.py:668-684, here taken through the softcap as well) and
 * scale = scale_grad * (scale_dev ? scale_dev[0] : 1). Ignored rows get a
 * zero row, out-of-range targets a NaN row.
 * Replaces kernels/ce_fused.py:490-522 (cross_entropy_bwd_tiny_hip).
 */
int ak_ce_bwd_tiny(const void* logits, const int64_t* targets,
                   const float* row_max, const float* row_sum, void* grad_logits,
                   int64_t rows, int64_t vocab, int64_t ld_logits, int64_t ld_grad,
                   float softcap, int64_t ignore_index, float label_smoothing,
                   float scale_grad, float z_loss_weight, const float* scale_dev,
                   int dtype, void* stream);

/*
 * denom[0] = max(1, #rows with targets[r] != ignore_index), denom[1] =
 * 1 / denom[0], fp32 on the device. One workgroup, integer count.
 * Replaces the host-side valid_mask.sum().clamp(min=1) and .item() of
 * kernels/ce_fused.py:590-605.
 */
int ak_ce_count_valid(const int64_t* targets, int64_t rows, int64_t ignore_index,
                      float* denom, void* stream);

/*
 * loss[0] = (sum over counted rows of losses[r] + z_loss_weight * lse[r]^2)
 *           / max(1, #counted rows)
 * n_valid[0] (nullable, int64) = #counted rows. Summed in a fixed order in
 * one workgroup (deterministic). lse may be NULL when z_loss_weight is 0.
 * Replaces the masked mean and z-loss of kernels/ce_fused.py:611-626.
 */
int ak_ce_mean(const float* losses, const float* lse, const int64_t* targets,
               int64_t rows, int64_t ignore_index, float z_loss_weight,
               float* loss, int64_t* n_valid, void* stream);

/*
 * Fused lm-head + cross-entropy forward: logits = hidden @ weight^T are
 * produced tile by tile on the matrix cores and folded into an online
 * logsumexp; they are never written to memory.
 *   lse[i]    = logsumexp_j(hidden[i] . weight[j])          (all rows)
 *   losses[i] = lse[i] - logit[i, target[i]]  or 0 if ignored (nullable)
 *   loss[0]   = sum(losses) / max(1, #non-ignored rows)
 *   n_valid[0]= #non-ignored rows (nullable, int64)
 * Replaces the per-chunk F.linear + cross_entropy_fwd_hip loop of
 * kernels/hip/chunked_linear_cross_entropy.py:55-148 (forward value and the
 * logsumexp side output). Only dtype AK_DTYPE_BF16 and AK_DTYPE_F16 are
 * accepted; d must be a multiple of 64, the rows of hidden and weight
 * 16-byte aligned and their pitches below 2^23 elements. workspace must
 * hold ak_lmhead_ce_workspace_bytes() bytes. logit[i, target[i]] is
 * computed as its own fp32-accumulated dot product. softcap > 0 replaces
 * every logit z by softcap * tanh(z / softcap) before the logsumexp and the
 * target term (the logit_softcap of kernels/ce_fused.py:236-260 and
 * chunked_linear_cross_entropy.py:20, 185); 0 disables it.
 * label_smoothing a in [0, 1] gives losses[i] = lse[i] - (1 - a) logit[i,
 * target[i]] - a mean_j(logit[i, j]) (kernels/ce_fused.py:29, :250-256);
 * 0 disables it.
 */
size_t ak_lmhead_ce_workspace_bytes(int64_t n_rows, int64_t vocab);
int ak_lmhead_ce_fwd(const void* hidden, const void* weight, const int64_t* targets,
                     float* loss, float* lse, float* losses, int64_t* n_valid,
                     void* workspace, size_t workspace_bytes,
                     int64_t n_rows, int64_t vocab, int64_t d,
                     int64_t ld_h, int64_t ld_w, int64_t ignore_index,
                     float softcap, float label_smoothing, int dtype, void* stream);

/*
 * Fused lm-head + cross-entropy backward, first half: the gradient of the
 * mean loss with respect to the logits, written without materialising the
 * logits first:
 *   grad_logits[i, v] = (softmax(hidden[i] . weight^T)[v] - [v == target[i]])
 *                       * grad_loss[0] / denom[0]
 * (0 for ignored rows, NaN for targets outside [0, vocab)). The logits are
 * recomputed tile by tile on the matrix cores from lse (the forward's
 * logsumexp output) and converted in registers; the target entries come from
 * fp32 dot products. grad_hidden = grad_logits @ weight and
 * grad_weight = grad_logits^T @ hidden are then plain GEMMs. Replaces the
 * per-chunk F.linear + cross_entropy_bwd_tiny_hip of
 * kernels/hip/chunked_linear_cross_entropy.py:150-175 (forward-side
 * gradient :97-132). grad_loss and denom are device pointers (no host
 * synchronisation). Same shape rules as ak_lmhead_ce_fwd; ld_gl >= vocab,
 * element type dtype (16-byte stores when ld_gl is a multiple of 8 and
 * grad_logits is 16-byte aligned, element stores otherwise). Only the first
 * vocab entries of each row are written. With softcap > 0 the gradient is
 * taken through the softcap (times 1 - tanh^2(z / softcap)), lse being the
 * forward's logsumexp of the capped logits. label_smoothing a replaces
 * softmax - one_hot by softmax - (1 - a) one_hot - a / vocab
 * (kernels/ce_fused.py:455-466).
 */
int ak_lmhead_ce_bwd(const void* hidden, const void* weight, const int64_t* targets,
                     const float* lse, const float* grad_loss, const float* denom,
                     void* grad_logits, int64_t ld_gl,
                     int64_t n_rows, int64_t vocab, int64_t d,
                     int64_t ld_h, int64_t ld_w, int64_t ignore_index,
                     float softcap, float label_smoothing, int dtype, void* stream);

/*
 * ak_lmhead_ce_bwd over the vocab columns [v_begin, v_begin + v_count) of a
 * vocab-entry problem: grad_logits holds v_count columns (ld_gl >= v_count),
 * column j being vocab entry v_begin + j; weight is the full [vocab, d]
 * matrix. Targets, the NaN rule for targets outside [0, vocab) and label
 * smoothing's a / vocab refer to the full vocabulary. A caller walks the
 * vocabulary in ranges so that only a [n_rows, v_count] slice of the
 * gradient exists at a time; each range's grad_weight rows are then a
 * complete GEMM and grad_hidden a sum over ranges. Same reference interface
 * as ak_lmhead_ce_bwd (kernels/hip/chunked_linear_cross_entropy.py:97-132,
 * which bounds the materialised gradient by chunking rows); ak_lmhead_ce_bwd
 * is this entry point with the range [0, vocab).
 */
int ak_lmhead_ce_bwd_range(const void* hidden, const void* weight, const int64_t* targets,
                           const float* lse, const float* grad_loss, const float* denom,
                           void* grad_logits, int64_t ld_gl, int64_t n_rows, int64_t vocab,
                           int64_t v_begin, int64_t v_count, int64_t d, int64_t ld_h,
                           int64_t ld_w, int64_t ignore_index, float softcap,
                           float label_smoothing, int dtype, void* stream);

/*
 * Gradient GEMMs of the lm-head + CE backward, from the dlogits written by
 * ak_lmhead_ce_bwd / ak_lmhead_ce_bwd_range (hand-written MFMA kernels,
 * fp32 accumulation). They replace the two torch.mm calls of the
 * reference's backward, kernels/hip/chunked_linear_cross_entropy.py:121-132
 * (grad_hidden = grad_logits @ weight, grad_weight = grad_logits^T @ hidden).
 *   grad_logits : [n_rows, ld_gl] of dtype; columns [0, vocab) hold the
 *                 gradient, columns [vocab, round_up(vocab, 64)) must be zero
 *                 (ld_gl >= round_up(vocab, 64), a multiple of 8, < 2^23,
 *                 every row readable to ld_gl)
 *   weight      : [vocab, d] rows of ld_w (the vocab range's rows)
 *   hidden      : [n_rows, d] rows of ld_h
 *   d           : multiple of 64; ld_w, ld_h >= d, multiples of 8, < 2^23
 *   out_mode    : 0 store in dtype, 1 store fp32, 2 add into fp32 (sums over
 *                 vocab ranges)
 *   workspace   : >= ak_lmhead_grad_workspace_bytes(n_rows, vocab, d) bytes
 *                 (fp32 partial tiles of K-split work; 0 when none is split),
 *                 16-byte aligned. The partial sums are added in a fixed order:
 *                 results are bitwise reproducible.
 * dtype: AK_DTYPE_BF16 or AK_DTYPE_F16.
 */
size_t ak_lmhead_grad_workspace_bytes(int64_t n_rows, int64_t vocab, int64_t d);

/* grad_hidden[t, :] = sum_v grad_logits[t, v] weight[v, :]; grad_hidden
 * [n_rows, d] rows of ld_gh (>= d). */
int ak_lmhead_grad_hidden(const void* grad_logits, int64_t ld_gl, const void* weight,
                          int64_t ld_w, void* grad_hidden, int64_t ld_gh, int64_t n_rows,
                          int64_t vocab, int64_t d, int out_mode, void* workspace,
                          size_t workspace_bytes, int dtype, void* stream);

/* grad_weight[v, :] = sum_t grad_logits[t, v] hidden[t, :]; grad_weight
 * [vocab, d] rows of ld_gw (>= d). */
int ak_lmhead_grad_weight(const void* grad_logits, int64_t ld_gl, const void* hidden,
                          int64_t ld_h, void* grad_weight, int64_t ld_gw, int64_t n_rows,
                          int64_t vocab, int64_t d, int out_mode, void* workspace,
                          size_t workspace_bytes, int dtype, void* stream);

/*
 * Mamba-1 selective scan forward (selective_scan_fn semantics).
 * Replaces selective_scan_cuda.fwd, external/mamba/csrc/selective_scan/
 * selective_scan.cpp:227-335, as called by
 * external/mamba/mamba_ssm/ops/selective_scan_interface.py:23-56; results
 * follow selective_scan_ref (selective_scan_interface.py:115-181) with fp32
 * state.
 *   u, z, out : [batch, dim, seqlen], element type u_dtype, last dim contiguous
 *   delta     : [batch, dim, seqlen], element type delta_dtype
 *   A         : [dim, dstate], a_dtype AK_DTYPE_F32 (real) or AK_DTYPE_C64
 *               (the reference's complex weights, selective_scan.cpp:236-240,
 *               selective_scan_interface.py:140-145, :173-174: complex state,
 *               y = 2 Re sum_n h C + D u); with C64 the state stride is 1 and
 *               A_dim_stride counts complex elements, and everything below
 *               marked "complex" applies (see the complex notes at the end)
 *   B, C      : variable: [batch, ngroups, dstate, seqlen], element type
 *               bc_dtype (strides batch / group / state);
 *               with AK_SCAN_B_CONST / AK_SCAN_C_CONST in bc_flags:
 *               input-independent [dim, dstate] fp32 (the reference's
 *               !is_variable_B / !is_variable_C, selective_scan.cpp:115-121):
 *               group_stride is then the dim stride, state_stride the state
 *               stride, batch_stride is ignored
 *   D, delta_bias : [dim] fp32 or NULL;  z may be NULL
 *   last_state: [batch, dim, dstate] fp32 or NULL
 *   out_prez  : y + D u before the gate, like out (strides of out), or NULL
 *               (the reference binding's `out` when z is given)
 *   chunk_states: [batch, dim, ceil(seqlen / 2048), dstate, 2] fp32 or NULL:
 *               per 2048-step chunk, the scan's running prefix from step 0 to
 *               the chunk's last step, (prod exp(delta' A), h) per state (the
 *               reference binding's `x`, selective_scan.cpp:307-313)
 *   checkpoints: [batch, ceil(seqlen / 16), dim, dstate] fp32 or NULL: the
 *               state before every 16-step block, for ak_selective_scan_bwd
 *               to restart from instead of re-running the forward (training
 *               keeps them; the reference's backward recomputes from `x`)
 * Strides are in elements. dim must be a multiple of ngroups; dstate <= 256
 * (the reference binding's limit, selective_scan.cpp:262). dstate <= 16 with
 * variable B / C runs the specialised kernels, everything else the general
 * ones.
 * Complex A (AK_DTYPE_C64; complex64 = interleaved fp32 re, im): a variable
 * B / C is real [batch, ngroups, dstate, 2 seqlen] in bc_dtype with the
 * (re, im) pair of step l at 2 l, 2 l + 1 (selective_scan.cpp:270-276); a
 * constant one is complex64 [dim, dstate] (strides in complex elements);
 * last_state is complex64 [batch, dim, dstate], chunk_states complex64
 * [batch, dim, ceil(seqlen / 2048), dstate, 2], checkpoints complex64
 * [batch, ceil(seqlen / 16), dim, dstate].
 */
int ak_selective_scan_fwd(const void* u, const void* delta, const float* A,
                          const void* B, const void* C, const float* D,
                          const void* z, const float* delta_bias,
                          void* out, float* last_state, void* out_prez, float* chunk_states,
                          float* checkpoints,
                          int64_t batch, int64_t dim, int64_t seqlen,
                          int64_t dstate, int64_t ngroups,
                          int64_t u_batch_stride, int64_t u_dim_stride,
                          int64_t delta_batch_stride, int64_t delta_dim_stride,
                          int64_t A_dim_stride,
                          int64_t B_batch_stride, int64_t B_group_stride, int64_t B_state_stride,
                          int64_t C_batch_stride, int64_t C_group_stride, int64_t C_state_stride,
                          int64_t z_batch_stride, int64_t z_dim_stride,
                          int64_t out_batch_stride, int64_t out_dim_stride,
                          int delta_softplus, int bc_flags,
                          int u_dtype, int delta_dtype, int bc_dtype, int a_dtype, void* stream);

/*
 * Mamba-1 selective scan backward: every input gradient of
 * ak_selective_scan_fwd's output given dout. Replaces selective_scan_cuda.bwd,
 * external/mamba/csrc/selective_scan/selective_scan.cpp:339-490, as called by
 * external/mamba/mamba_ssm/ops/selective_scan_interface.py:59-83 (its
 * recompute_out_z option and the saved chunk states x are not needed: the
 * states are recomputed here, or taken from the forward's checkpoints).
 *   inputs, bc_flags and a_dtype as for ak_selective_scan_fwd; dout
 *               [batch, dim, seqlen] in u_dtype
 *   du, dz    : contiguous [batch, dim, seqlen], u_dtype (dz only with z)
 *   ddelta    : contiguous [batch, dim, seqlen], delta_dtype
 *   dA        : contiguous [dim, dstate] fp32
 *   dB, dC    : variable: contiguous [batch, ngroups, dstate, seqlen] in
 *               bc_dtype (summed in fp32 and rounded once, as the reference's
 *               fp32 accumulation and dB.to(B.dtype()), selective_scan.cpp:461,
 *               :488); constant: contiguous [dim, dstate] fp32
 *   dD, ddelta_bias : [dim] fp32, required when D / delta_bias are given
 *   checkpoints, out_prez : NULL, or the forward's `checkpoints` and (with z)
 *               its `out_prez` as a contiguous [batch, dim, seqlen] tensor.
 *               Given, the backward skips its re-run of the forward: it
 *               restarts from the saved states, which it only reads, and
 *               computes dz from out_prez. Every gradient but dz is then
 *               bitwise the same; dz uses the stored (rounded) pre-gate
 *               output, as the reference's backward does with its `out`.
 * workspace: ak_selective_scan_bwd_workspace_bytes(...) bytes (saved states
 * every 16 steps and the partial sums of dB / dC / dA / dD / ddelta_bias,
 * reduced in a fixed order: results are bitwise reproducible; large
 * whole-tile shapes, with batch x ngroups x channels-per-group / 32 >= 256,
 * group 32 channels per partial dB / dC row, a choice fixed by the shape
 * alone, so the bits do not depend on the device's compute-unit count).
 * Complex A: dA is complex64 [dim, dstate]; a variable dB / dC is real
 * [batch, ngroups, dstate, 2 seqlen] in bc_dtype, a constant one complex64
 * [dim, dstate]; checkpoints are the forward's complex ones; complex
 * gradients are packed as dL/dRe + i dL/dIm (torch autograd's convention).
 * The workspace size is ak_selective_scan_bwd_workspace_bytes(..., bc_flags |
 * AK_SCAN_A_COMPLEX); without saved states it holds the re-run forward's
 * states and pre-gate output, and a variable dB / dC takes one fp32 partial
 * row per 4 channels of a group (4 * 2 seqlen * dstate * ngroups * batch *
 * dim / ngroups / 4 bytes each).
 */
size_t ak_selective_scan_bwd_workspace_bytes(int64_t batch, int64_t dim, int64_t seqlen,
                                             int64_t dstate, int64_t ngroups, int bc_flags);
int ak_selective_scan_bwd(const void* u, const void* delta, const float* A,
                          const void* B, const void* C, const float* D,
                          const void* z, const float* delta_bias, const void* dout,
                          void* du, void* ddelta, float* dA, void* dB, void* dC,
                          float* dD, void* dz, float* ddelta_bias,
                          const float* checkpoints, const void* out_prez,
                          void* workspace, size_t workspace_bytes,
                          int64_t batch, int64_t dim, int64_t seqlen,
                          int64_t dstate, int64_t ngroups,
                          int64_t u_batch_stride, int64_t u_dim_stride,
                          int64_t delta_batch_stride, int64_t delta_dim_stride,
                          int64_t A_dim_stride,
                          int64_t B_batch_stride, int64_t B_group_stride, int64_t B_state_stride,
                          int64_t C_batch_stride, int64_t C_group_stride, int64_t C_state_stride,
                          int64_t z_batch_stride, int64_t z_dim_stride,
                          int64_t dout_batch_stride, int64_t dout_dim_stride,
                          int delta_softplus, int bc_flags,
                          int u_dtype, int delta_dtype, int bc_dtype, int a_dtype, void* stream);

/*
 * Diagonal linear recurrence over [batch, seqlen, d_inner] fp32 tensors:
 *   s[t] = dA[t] * s[t-1] + dBx[t];  y[t] = C[t] * s[t] + D * x[t]
 * Replaces kernels/hip/selective_scan.py:165-201 (selective_scan_hip).
 */
int ak_diag_scan_fwd(const float* dA, const float* dBx, const float* C,
                     const float* D, const float* x, float* y,
                     int64_t batch, int64_t seqlen, int64_t d_inner, void* stream);

/*
 * Backward of the diagonal recurrence of ak_diag_scan_fwd, all fp32
 * [batch, seqlen, d_inner] (grad_D [d_inner]):
 *   grad_C[t] = gy[t] * state[t];  g += gy[t] * C[t];  grad_dA[t] = g * state[t-1];
 *   grad_dBx[t] = g;  g *= dA[t];  grad_x[t] = gy[t] * D;  grad_D = sum_{b,t} gy * x
 * Replaces kernels/hip/selective_scan_backward.py:393-421 (kernel_fn) and its
 * kernels :72-311 (the gradient of kernels/hip/_torch_ops.py:346-386).
 * grad_C doubles as the recomputed-state buffer (no extra allocation).
 * workspace: ak_diag_scan_bwd_workspace_bytes(batch, d_inner) bytes for the
 * per-(batch, channel) partial sums of grad_D, reduced in batch order.
 */
size_t ak_diag_scan_bwd_workspace_bytes(int64_t batch, int64_t d_inner);
int ak_diag_scan_bwd(const float* dA, const float* dBx, const float* C, const float* D,
                     const float* x, const float* grad_y,
                     float* grad_dA, float* grad_dBx, float* grad_C, float* grad_D,
                     float* grad_x, void* workspace, size_t workspace_bytes,
                     int64_t batch, int64_t seqlen, int64_t d_inner, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AUTOKERNEL_MI355X_H */
