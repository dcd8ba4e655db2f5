"""Linear (lm-head) + cross-entropy without materialised logits, gfx950.

Drop-in for the reference module ``kernels/hip/chunked_linear_cross_entropy.py``
(``ChunkedLinearCrossEntropyLoss`` :178-229, ``_ChunkedLinearCrossEntropy``
:50-175): same constructor arguments, same ``forward(hidden, weight,
targets)`` contract, autograd for ``hidden`` and ``weight``.

Forward (bf16/fp16, any hidden size ``d``; any softcap and label
smoothing): one fused kernel,
``ak_lmhead_ce_fwd`` (``csrc/lmhead_ce.hip``), computes ``hidden @ weight^T``
tile by tile on the matrix cores and folds each tile into an online
logsumexp, so the ``[N, V]`` logits never exist in memory and there is no
host synchronisation. It returns the mean loss over non-ignored rows and
the per-row logsumexp (used by the z-loss and by the backward). With
``softcap`` > 0 every logit ``z`` becomes ``softcap * tanh(z / softcap)`` in
the kernel's epilogue (the reference's ``logit_softcap``), and the tile
partials use ``softcap`` as their offset (no max pass). With
``label_smoothing`` a the loss is ``lse - (1 - a) z_t - a mean(z)``; the
tile epilogue then also sums the (capped) logits of each token.

The kernels take ``d`` in 64-wide blocks: a ``d`` that is not a multiple
of 64 is zero-extended on the way in (exact: the extra columns add zeros to
every dot product) and the gradients are cut back to ``d`` columns.

For fp32 inputs the forward runs the reference's row-chunked algorithm: per
``chunk_size`` rows a GEMM (``torch.nn.functional.linear``) feeds the gfx950
CE row kernel.

Backward (the fused forward's conditions): ``ak_lmhead_ce_bwd``
recomputes the logits tile by tile on the matrix cores from the saved
logsumexp and writes ``dL/dlogits`` (softmax minus one-hot, times the
upstream gradient over the counted rows, times ``1 - tanh^2`` under the
softcap, less ``a / vocab`` under label smoothing) directly from registers in the
input dtype; the device scalars stay on the device (no host sync). Then
``grad_hidden = dlogits @ W`` and ``grad_W = dlogits^T @ h`` run as two
hand-written MFMA GEMMs with fp32 accumulation (``ak_lmhead_grad_hidden``,
``ak_lmhead_grad_weight``, ``csrc/lmhead_grad_gemm.hip``): dlogits is read
in place, token-major, by both (the transposed operand through gfx950's
transposing LDS reads). The vocabulary is walked in ranges whose
``dlogits`` slice ``[n_rows, width]`` stays under ``GRAD_LOGITS_BUDGET``
bytes (``ak_lmhead_ce_bwd_range``; whole 256-row vocab tiles, the ranges as
even as whole rounds of the tile kernel allow: ``_vocab_ranges``). Each range's ``grad_W`` rows are one complete GEMM rounded
once to the weight dtype; ``grad_hidden`` is summed over the ranges in an
fp32 buffer (the GEMM's add-into-fp32 output) and rounded once at the end.
The default budget (4 GiB) keeps the C4 shape in one range (8192 x 50304
bf16 = 824 MB, 0.3% of the 288 GB of HBM); lower it where memory matters
more than time.
For fp32 inputs, per row chunk the logits are recomputed with a GEMM and
turned into ``dL/dlogits`` by the CE row kernel from the saved logsumexp
(the upstream gradient over the counted rows as a device scalar: no host
sync, where the reference read both with ``.item()``), then
``grad_hidden = dlogits @ W`` and ``grad_W += dlogits^T @ h`` (fp32
accumulation), as in the reference (``:97-132``, ``:150-175``). An empty
batch gives a zero loss and empty / zero gradients. As in the reference, the z-loss term
contributes to the returned loss only, not to the gradient.

``chunk_size`` is the row-chunk of the GEMM paths; the fused forward tiles
the vocabulary itself. Inputs keep their dtype (the reference coerced
everything to fp16).
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from kernels.hip import _lib


def _fused_ok(hidden: torch.Tensor, weight: torch.Tensor, softcap: float,
              label_smoothing: float) -> bool:
    """Whether the matrix-core kernels take the call: half-precision inputs of
    one dtype and a finite softcap / smoothing in range. Any hidden size and
    alignment qualify (``_kernel_operands`` pads and realigns)."""
    return (0.0 <= softcap < float("inf") and 0.0 <= label_smoothing <= 1.0
            and hidden.dtype in (torch.bfloat16, torch.float16) and weight.dtype == hidden.dtype)


# The tile kernels consume the hidden dimension in 64-wide blocks.
_K_BLOCK = 64


def _kernel_operands(hidden: torch.Tensor, weight: torch.Tensor):
    """``(hidden, weight)`` as the fused kernels need them: contiguous,
    16-byte aligned, hidden size a multiple of 64. A hidden size that is not
    is zero-extended (both operands get the same zero columns), which adds
    exact zeros to every logit's dot product, so the logits and both
    gradients' first ``d`` columns are those of the unpadded problem."""
    d = hidden.shape[1]
    dk = -(-d // _K_BLOCK) * _K_BLOCK
    if dk != d:
        hp = hidden.new_zeros((hidden.shape[0], dk))
        hp[:, :d] = hidden
        wp = weight.new_zeros((weight.shape[0], dk))
        wp[:, :d] = weight
        return hp, wp
    hidden, weight = hidden.contiguous(), weight.contiguous()
    if hidden.data_ptr() % 16:
        hidden = hidden.clone()
    if weight.data_ptr() % 16:
        weight = weight.clone()
    return hidden, weight


def lmhead_ce_forward(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                      ignore_index: int = -100, return_losses: bool = False,
                      softcap: float = 0.0, label_smoothing: float = 0.0):
    """Fused forward: returns ``(loss, lse, n_valid)`` (+ per-row losses).

    ``loss`` is a 0-d fp32 tensor (mean over non-ignored rows), ``lse`` fp32
    ``[N]``, ``n_valid`` a 1-element int64 tensor. No host synchronisation.
    """
    _lib.require_device(hidden, weight, targets)
    hidden, weight = _kernel_operands(hidden, weight)
    targets = targets.contiguous().to(torch.int64)
    n = hidden.shape[0]
    dev = hidden.device
    loss = torch.empty((), dtype=torch.float32, device=dev)
    lse = torch.empty(n, dtype=torch.float32, device=dev)
    n_valid = torch.empty(1, dtype=torch.int64, device=dev)
    losses = torch.empty(n, dtype=torch.float32, device=dev) if return_losses else None
    if n == 0:  # an empty batch: no counted rows, loss 0 (the mean over max(1, 0) rows)
        loss.zero_()
        n_valid.zero_()
        return (loss, lse, n_valid, losses) if return_losses else (loss, lse, n_valid)
    ws = torch.empty(_lib.lmhead_ce_workspace_bytes(n, weight.shape[0]), dtype=torch.uint8, device=dev)
    _lib.lmhead_ce(hidden, weight, targets, loss, lse, losses, n_valid, ws, ignore_index, softcap,
                   label_smoothing)
    if return_losses:
        return loss, lse, n_valid, losses
    return loss, lse, n_valid


# Largest dlogits slice (bytes) the fused backward materialises at once.
GRAD_LOGITS_BUDGET = 4 << 30
# Row pitch padding of a range's slice (elements): keeps the pitch off powers
# of two, whose rows would all start in the same memory channels.
_RANGE_PAD = 64
# Vocab ranges are whole multiples of the tile kernel's vocab tile.
_VOCAB_TILE = 256


def _vocab_ranges(n: int, vocab: int, elem: int, cus: int):
    """Vocab ranges ``[v0, v1)`` whose dlogits slices (``n x (v1 - v0)``
    elements of ``elem`` bytes) fit ``GRAD_LOGITS_BUDGET``.

    The fewest ranges that fit, of whole vocab tiles, as even as the tile
    kernel allows: ranges of ``w`` tiles with the rest in the last one, ``w``
    a multiple of ``q``, where ``q`` vocab tiles times the ``ceil(n / 256)``
    token tiles is a multiple of the CU count (each launch then runs whole
    rounds of the persistent workgroups). ``w`` is the even share rounded
    down to a multiple of ``q`` if the last range then still fits, else
    rounded up if that fits, else the even share itself. Measured at C4
    (whole backward, one process): a 512 MB budget takes 96 + 100.5 tiles,
    632 MiB and 0-4% faster than 128 + 68.5 at 816 MiB; 256 MB takes
    48 + 48 + 48 + 52.5, 440 MiB at the same time as 64 + 64 + 64 + 4.5 at
    488 MiB; at 128 MB the even share of 29 tiles ran 5% slower than 32-tile
    ranges, which rounding up gives.
    """
    tiles = -(-vocab // _VOCAB_TILE)
    cap = max(1, min(tiles, GRAD_LOGITS_BUDGET // (n * elem * _VOCAB_TILE)))
    count = -(-tiles // cap)
    if count == 1:
        return [(0, vocab)]
    per = -(-tiles // count)
    q = cus // math.gcd(cus, -(-n // 256))
    down, up = per // q * q, -(-per // q) * q
    if down > 0 and tiles - (count - 1) * down <= cap:
        per = down
    elif up <= cap:
        per = up
    # count ranges of per tiles, the last one holding the rest: it is not
    # empty since (count - 1) * per < tiles, and it fits by the choice above
    cuts = [i * per * _VOCAB_TILE for i in range(count)] + [vocab]
    return [(cuts[i], cuts[i + 1]) for i in range(count)]


def lmhead_ce_backward(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                       lse: torch.Tensor, denom: torch.Tensor, grad_loss: torch.Tensor,
                       ignore_index: int = -100, need_hidden: bool = True,
                       need_weight: bool = True, softcap: float = 0.0,
                       label_smoothing: float = 0.0):
    """Fused backward of :func:`lmhead_ce_forward`'s mean loss.

    ``lse`` is the forward's logsumexp, ``denom`` the number of counted rows
    (a 0-d or 1-element fp32 tensor, clamped to >= 1) and ``grad_loss`` the
    upstream gradient of the loss, ``softcap`` and ``label_smoothing`` the
    forward's.
    Returns ``(grad_hidden, grad_weight)`` in the input dtype (``None`` where
    not requested).
    """
    _lib.require_device(hidden, weight, targets, lse, denom, grad_loss)
    d_in = hidden.shape[1]
    hidden, weight = _kernel_operands(hidden, weight)
    targets = targets.contiguous().to(torch.int64)
    n, d = hidden.shape
    vocab = weight.shape[0]
    if n == 0:
        return (torch.empty((0, d_in), dtype=hidden.dtype, device=hidden.device) if need_hidden else None,
                torch.zeros((vocab, d_in), dtype=weight.dtype, device=weight.device) if need_weight else None)
    g1 = grad_loss.reshape(1).to(torch.float32).contiguous()
    den1 = denom.reshape(1).to(torch.float32).contiguous()
    lse = lse.contiguous()
    # the CU count only shapes the plan (a CPU tensor reaches here only from
    # the tests' fake backend: MI355X's 256)
    cus = (torch.cuda.get_device_properties(hidden.device).multi_processor_count
           if hidden.device.type == "cuda" else 256)
    ranges = _vocab_ranges(n, vocab, hidden.element_size(), cus)
    width = max(v1 - v0 for v0, v1 in ranges)
    # each range's dlogits slice lives in a buffer whose pitch covers the
    # slice rounded up to 64 columns (the gradient GEMMs read whole 64-column
    # K blocks); a pitch off powers of two keeps the rows from all starting
    # in the same memory channels
    pitch = -(-width // 64) * 64
    if pitch & (pitch - 1) == 0:
        pitch += 64
    gp = torch.empty((n, pitch), dtype=hidden.dtype, device=hidden.device)
    ws_bytes = max(_lib.lmhead_grad_workspace_bytes(n, v1 - v0, d) for v0, v1 in ranges)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=hidden.device) if ws_bytes else None
    single = len(ranges) == 1
    grad_weight = torch.empty_like(weight) if need_weight else None
    if need_hidden:
        grad_hidden = torch.empty_like(hidden) if single else \
            torch.zeros((n, d), dtype=torch.float32, device=hidden.device)
    else:
        grad_hidden = None
    for v0, v1 in ranges:
        g = gp[:, :v1 - v0]  # lmhead_grad_hidden zeroes its K padding
        _lib.lmhead_ce_bwd_range(hidden, weight, targets, lse, g1, den1, g, v0, ignore_index,
                                 softcap, label_smoothing)
        if need_weight:
            _lib.lmhead_grad_weight(g, hidden, grad_weight[v0:v1], _lib.GEMM_OUT_DTYPE, ws)
        if need_hidden:
            _lib.lmhead_grad_hidden(g, weight[v0:v1], grad_hidden,
                                    _lib.GEMM_OUT_DTYPE if single else _lib.GEMM_OUT_F32_ADD, ws)
    if need_hidden and not single:
        grad_hidden = grad_hidden.to(hidden.dtype)
    if d != d_in:  # drop the zero extension of the hidden size
        grad_hidden = grad_hidden[:, :d_in].contiguous() if need_hidden else None
        grad_weight = grad_weight[:, :d_in].contiguous() if need_weight else None
    return grad_hidden, grad_weight


def _chunked_forward(hidden, weight, targets, chunk_size, softcap, ignore_index, label_smoothing):
    """Row-chunked GEMM + CE row kernel; returns (loss_sum, lse, n_valid float tensor)."""
    from kernels.ce_fused import _get_fwd_module
    mod = _get_fwd_module()
    n = hidden.shape[0]
    lse = torch.empty(n, dtype=torch.float32, device=hidden.device)
    loss_sum = torch.zeros((), dtype=torch.float32, device=hidden.device)
    for start in range(0, n, chunk_size):
        end = min(start + chunk_size, n)
        logits = F.linear(hidden[start:end], weight)
        t = targets[start:end]
        losses, lse_c, _, _, _ = mod.cross_entropy_fwd_hip(
            logits, t, float(softcap), int(ignore_index), float(label_smoothing), 0, 0, 1.0)
        lse[start:end] = lse_c
        loss_sum = loss_sum + (losses * (t != ignore_index).to(torch.float32)).sum()
    n_valid = (targets != ignore_index).sum().to(torch.float32).clamp(min=1.0)
    return loss_sum / n_valid, lse, n_valid


class _ChunkedLinearCrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, weight, targets, chunk_size, softcap, ignore_index,
                label_smoothing, z_loss_weight):
        targets = targets.contiguous().to(torch.int64)
        if _fused_ok(hidden, weight, softcap, label_smoothing):
            loss, lse, n_valid_i = lmhead_ce_forward(hidden, weight, targets, ignore_index,
                                                     softcap=float(softcap),
                                                     label_smoothing=float(label_smoothing))
            n_valid = n_valid_i.to(torch.float32).clamp(min=1.0).reshape(())
        else:
            loss, lse, n_valid = _chunked_forward(hidden.contiguous(), weight.contiguous(), targets,
                                                  chunk_size, softcap, ignore_index,
                                                  label_smoothing)
        if z_loss_weight > 0:
            valid = (targets != ignore_index).to(torch.float32)
            loss = loss + z_loss_weight * ((lse * valid).pow(2).sum() / n_valid)
        ctx.save_for_backward(hidden, weight, targets, lse, n_valid)
        ctx.fused = _fused_ok(hidden, weight, softcap, label_smoothing)
        ctx.chunk_size = int(chunk_size)
        ctx.softcap = float(softcap)
        ctx.ignore_index = int(ignore_index)
        ctx.label_smoothing = float(label_smoothing)
        return loss

    @staticmethod
    def backward(ctx, grad_output):
        hidden, weight, targets, lse, n_valid = ctx.saved_tensors
        need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if ctx.fused and (need_h or need_w):
            gh, gw = lmhead_ce_backward(hidden, weight, targets, lse, n_valid, grad_output,
                                        ctx.ignore_index, need_h, need_w, ctx.softcap,
                                        ctx.label_smoothing)
            return gh, gw, None, None, None, None, None, None
        grad_hidden = torch.empty_like(hidden) if need_h else None
        grad_weight = torch.zeros(weight.shape, dtype=torch.float32, device=weight.device) if need_w else None
        if need_h or need_w:
            # upstream gradient / #counted rows, on the device (no host sync)
            scale = (grad_output.detach().to(torch.float32).reshape(1) / n_valid.reshape(1)).contiguous()
            ones = torch.ones_like(lse)
            w = weight.contiguous()
            h = hidden.contiguous()
            n = h.shape[0]
            for start in range(0, n, ctx.chunk_size):
                end = min(start + ctx.chunk_size, n)
                logits = F.linear(h[start:end], w)
                # softmax = exp(x - lse) / 1: lse as the row max and 1 as the row sum
                glog = torch.empty_like(logits)
                _lib.ce_bwd_tiny(logits, targets[start:end], lse[start:end], ones[start:end], glog,
                                 ctx.softcap, ctx.ignore_index, ctx.label_smoothing, 1.0,
                                 scale_dev=scale)
                if need_h:
                    grad_hidden[start:end] = glog @ w
                if need_w:
                    grad_weight.addmm_(glog.t().to(torch.float32), h[start:end].to(torch.float32))
            if need_w:
                grad_weight = grad_weight.to(weight.dtype)
        return grad_hidden, grad_weight, None, None, None, None, None, None


class ChunkedLinearCrossEntropyLoss(nn.Module):
    """Drop-in for ``nn.Linear`` + ``nn.CrossEntropyLoss`` without materialised logits.

    Args:
        chunk_size: rows per chunk of the fp32 path's GEMMs (the half-precision
            kernels tile the problem themselves).
        softcap: logit softcap (0 = off).
        ignore_index: target value to mask (default -100).
        label_smoothing: alpha (0 = off).
        z_loss_weight: if > 0, adds ``z * mean(lse^2)`` over non-ignored rows.
    """

    def __init__(self, chunk_size: int = 512, softcap: float = 0.0, ignore_index: int = -100,
                 label_smoothing: float = 0.0, z_loss_weight: float = 0.0):
        super().__init__()
        self.chunk_size = int(chunk_size)
        self.softcap = float(softcap)
        self.ignore_index = int(ignore_index)
        self.label_smoothing = float(label_smoothing)
        self.z_loss_weight = float(z_loss_weight)

    def forward(self, hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
        if hidden.dim() == 3:
            b, t, d = hidden.shape
            hidden = hidden.reshape(b * t, d)
        if targets.dim() == 2:
            targets = targets.reshape(-1)
        _lib.require_device(hidden, weight, targets)
        if weight.dtype != hidden.dtype:
            weight = weight.to(hidden.dtype)
        return _ChunkedLinearCrossEntropy.apply(
            hidden, weight, targets, self.chunk_size, self.softcap, self.ignore_index,
            self.label_smoothing, self.z_loss_weight)
