"""Cross-entropy over materialised logits on gfx950 (MI355X).

Drop-in for the reference module ``kernels/ce_fused.py``: same public names
(``kernel_fn``, ``ce_full``, ``_CrossEntropyHIP``, ``_get_fwd_module``,
``_get_bwd_module``, the harness constants and ``HIP_FWD_SRC`` /
``HIP_BWD_SRC``), same arguments and the same loss / gradient semantics
(``ce_fused.py:557-785``):

* per row: ``lse = logsumexp(x)``, ``loss = lse - x[t]`` (label smoothing
  ``a``: ``lse - (1-a) x[t] - a mean(x)``; softcap: ``x = c tanh(x / c)``),
  ignored rows give loss 0 and a zero gradient row;
* scalar loss = sum over non-ignored rows / max(1, #non-ignored), plus
  ``w * sum(lse^2) / max(1, #non-ignored)`` with a z-loss weight ``w``;
* "fused" mode writes the gradient during the forward; "tiny" mode saves
  the row max / sum and recomputes the gradient in the backward.

Everything runs on the device in four small steps, with no host read in the
forward: ``ak_ce_count_valid`` counts the rows that take part,
``ak_ce_fwd`` computes the per-row results (and, in fused mode, the gradient
already scaled by 1 / count read from device memory), ``ak_ce_mean`` reduces
them in a fixed order, and ``ak_ce_bwd_tiny`` is the tiny-mode backward with
the upstream gradient taken from device memory. The z-loss gradient
``2 w lse p / count`` is part of both gradient kernels, so the z-loss works in
either mode and is taken through the softcap.

Differences from the reference, all deliberate: bf16 and fp32 logits run on
the GPU kernels in their own dtype (the reference cast bf16 to fp16 and sent
fp32 to PyTorch); an out-of-range target (neither in ``[0, V)`` nor
``ignore_index``) yields a NaN loss instead of an out-of-bounds read; the
tiny-mode gradient is scaled by 1 / #non-ignored rows (the gradient of the
returned mean; the reference scaled it by 1 / batch); a z-loss no longer
switches fused mode to tiny mode, and its gradient includes the softcap's
``1 - tanh^2`` factor.
"""

import os

import torch

from kernels.hip import _lib

KERNEL_TYPE = "cross_entropy"
BACKEND = "hip"

MODEL_SHAPES = {'batch': 4096, 'vocab': 32768}

TEST_SIZES = [
    ("model_primary", {'batch': 4096, 'vocab': 32768}),
    ("model_half", {'batch': 2048, 'vocab': 16384}),
    ("model_double", {'batch': 8192, 'vocab': 65536}),
]

TOLERANCES = {'float16': {'atol': 0.01, 'rtol': 0.01}, 'bfloat16': {'atol': 0.02, 'rtol': 0.02},
              'float32': {'atol': 1e-05, 'rtol': 1e-05}}


def FLOPS_FN(s):
    return 4 * s["batch"] * s["vocab"]


def BYTES_FN(s, dt_bytes):
    return (s["batch"] * s["vocab"] + s["batch"]) * dt_bytes


# Source locations (the reference kept the source text in these names).
HIP_FWD_SRC = os.path.join(_lib.CSRC_DIR, "ce_rows.hip")
HIP_BWD_SRC = HIP_FWD_SRC


# A target value no int64 row holds: "no ignore_index".
_NO_IGNORE = -(2 ** 63)


def _row_problem(logits: torch.Tensor, targets: torch.Tensor):
    """Checks and brings logits to a ``[rows, vocab]`` view the row kernels take
    and targets to contiguous int64."""
    _lib.require_device(logits, targets)
    if logits.dim() != 2:
        raise ValueError("logits must be [batch, vocab]")
    _lib.dtype_code(logits.dtype)
    tg = targets.reshape(-1).contiguous().to(torch.int64)
    if tg.numel() != logits.size(0):
        raise ValueError(f"{tg.numel()} targets for {logits.size(0)} rows")
    return _lib.as_rows(logits, logits.size(1)), tg


class _FwdModule:
    """Stands where the reference's JIT-built forward module stood."""

    @staticmethod
    def cross_entropy_fwd_hip(logits, targets, softcap, ignore_index, label_smoothing,
                              write_grad, save_max_sum, scale_grad):
        """Returns ``[losses, lse, row_max, row_sum, grad_logits]`` (None where not requested)."""
        logits, targets = _row_problem(logits, targets)
        B = logits.size(0)
        f32 = dict(dtype=torch.float32, device=logits.device)
        losses = torch.empty(B, **f32)
        lse = torch.empty(B, **f32)
        row_max = torch.empty(B, **f32) if save_max_sum else None
        row_sum = torch.empty(B, **f32) if save_max_sum else None
        grad = torch.empty(logits.shape, dtype=logits.dtype, device=logits.device) if write_grad else None
        if B:
            _lib.ce_fwd(logits, targets, losses, lse, row_max, row_sum, grad, float(softcap),
                        int(ignore_index), float(label_smoothing), float(scale_grad))
        return [losses, lse, row_max, row_sum, grad]


class _BwdModule:
    @staticmethod
    def cross_entropy_bwd_tiny_hip(logits, targets, row_maxes, row_sums, softcap, ignore_index,
                                   label_smoothing, scale_grad):
        _lib.require_device(logits, targets, row_maxes, row_sums)
        logits = _lib.as_rows(logits, logits.size(-1))
        grad = torch.empty(logits.shape, dtype=logits.dtype, device=logits.device)
        if logits.size(0):
            _lib.ce_bwd_tiny(logits, targets.contiguous().to(torch.int64),
                             row_maxes.float().contiguous(), row_sums.float().contiguous(), grad,
                             float(softcap), int(ignore_index), float(label_smoothing),
                             float(scale_grad))
        return grad


_fwd_module = _FwdModule()
_bwd_module = _BwdModule()


def _get_fwd_module():
    return _fwd_module


def _get_bwd_module():
    return _bwd_module


class _CrossEntropyHIP(torch.autograd.Function):
    """Mean CE over the counted rows, with the gradient either written by the
    forward (``mode="fused"``) or recomputed from the saved row statistics
    (``mode="tiny"``).

    Arguments and return values are those of ``kernels/ce_fused.py:557-578``:
    ``(logits, targets, softcap, ignore_index, label_smoothing, mode,
    return_z, z_loss_weight)`` -> ``loss``, or ``(loss, lse)`` with
    ``return_z``. ``ignore_index=None`` counts every row.
    """

    @staticmethod
    def forward(ctx, logits, targets, softcap, ignore_index, label_smoothing, mode, return_z,
                z_loss_weight=0.0):
        rows2d, tg = _row_problem(logits, targets)
        n = rows2d.size(0)
        ign = _NO_IGNORE if ignore_index is None else int(ignore_index)
        params = (float(softcap), ign, float(label_smoothing), float(z_loss_weight))
        on_dev = dict(dtype=torch.float32, device=rows2d.device)
        losses, lse = torch.empty(n, **on_dev), torch.empty(n, **on_dev)
        # [max(1, #counted rows), its reciprocal], never read on the host
        denom = _lib.ce_count_valid(tg, ign)
        keep_grad = mode == "fused"
        if keep_grad:
            grad, row_max, row_sum = torch.empty(rows2d.shape, dtype=rows2d.dtype,
                                                 device=rows2d.device), None, None
        else:
            grad, row_max, row_sum = None, torch.empty(n, **on_dev), torch.empty(n, **on_dev)
        if n:
            _lib.ce_fwd(rows2d, tg, losses, lse, row_max, row_sum, grad, params[0], ign, params[2],
                        1.0, scale_dev=denom[1:], z_loss_weight=params[3])
        loss = _lib.ce_mean(losses, lse, tg, ign, params[3])

        ctx.params = params
        ctx.keep_grad = keep_grad
        if keep_grad:
            ctx.save_for_backward(grad)
        else:
            ctx.save_for_backward(rows2d, tg, row_max, row_sum, denom)
        ctx.mark_non_differentiable(lse)
        return (loss, lse) if return_z else loss

    @staticmethod
    def backward(ctx, grad_loss, *unused):
        softcap, ign, ls, zw = ctx.params
        if ctx.keep_grad:
            (grad,) = ctx.saved_tensors
            # The saved gradient already carries 1 / #counted rows; the
            # upstream gradient is applied on the device (a product with 1.0
            # returns the saved bits), so the backward never waits for the GPU.
            grad = grad * grad_loss.detach().to(grad.dtype)
        else:
            rows2d, tg, row_max, row_sum, denom = ctx.saved_tensors
            # upstream gradient / #counted rows, kept on the device
            scale = grad_loss.detach().to(torch.float32).reshape(1) * denom[1:]
            grad = torch.empty(rows2d.shape, dtype=rows2d.dtype, device=rows2d.device)
            if rows2d.size(0):
                _lib.ce_bwd_tiny(rows2d, tg, row_max, row_sum, grad, softcap, ign, ls, 1.0, zw,
                                 scale_dev=scale)
        return (grad,) + (None,) * 7


def kernel_fn(logits: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    """Mean cross-entropy; matches ``reference.cross_entropy_ref`` (ignore_index -100)."""
    if logits.requires_grad and torch.is_grad_enabled():
        return _CrossEntropyHIP.apply(logits, targets, 0.0, -100, 0.0, "fused", False, 0.0)
    rows2d, tg = _row_problem(logits, targets)
    on_dev = dict(dtype=torch.float32, device=rows2d.device)
    losses = torch.empty(rows2d.size(0), **on_dev)
    lse = torch.empty(rows2d.size(0), **on_dev)
    if rows2d.size(0):
        _lib.ce_fwd(rows2d, tg, losses, lse, None, None, None, 0.0, -100, 0.0, 1.0)
    return _lib.ce_mean(losses, None, tg, -100)


def ce_full(logits: torch.Tensor, targets: torch.Tensor, *, softcap: float = 0.0,
            ignore_index: int = -100, label_smoothing: float = 0.0, mode: str = "fused",
            return_z: bool = False, z_loss_weight: float = 0.0):
    """Full-featured CE; arguments as ``kernels/ce_fused.py:726-785`` of the reference."""
    _lib.require_device(logits, targets)
    if mode not in ("fused", "tiny"):
        raise ValueError(f"mode must be 'fused' or 'tiny', got {mode!r}")
    return _CrossEntropyHIP.apply(logits, targets, softcap, ignore_index, label_smoothing, mode,
                                  return_z, float(z_loss_weight))
