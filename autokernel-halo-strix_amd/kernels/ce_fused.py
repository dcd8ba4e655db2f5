"""Cross-entropy over materialised logits on gfx950 (MI355X).

Drop-in for the reference module ``kernels/ce_fused.py``: same public names
(``kernel_fn``, ``ce_full``, ``_CrossEntropyHIP``, ``_get_fwd_module``,
``_get_bwd_module``, the harness constants and ``HIP_FWD_SRC`` /
``HIP_BWD_SRC``), same arguments and the same loss / gradient semantics
(``ce_fused.py:557-785``):

* per row: ``lse = logsumexp(x)``, ``loss = lse - x[t]`` (label smoothing
  ``a``: ``lse - (1-a) x[t] - a mean(x)``; softcap: ``x = c tanh(x / c)``),
  ignored rows give loss 0 and a zero gradient row;
* scalar loss = sum over non-ignored rows / max(1, #non-ignored);
* "fused" mode writes the pre-scaled gradient during the forward; "tiny"
  mode saves row max / sum and recomputes the gradient in the backward;
  ``z_loss_weight > 0`` forces tiny mode and adds ``w * mean(lse^2)``.

The kernels are ``ak_ce_fwd`` / ``ak_ce_bwd_tiny`` (``csrc/ce_rows.hip``).
Differences from the reference, all deliberate: bf16 and fp32 logits run on
the GPU kernels in their own dtype (the reference cast bf16 to fp16 and sent
fp32 to PyTorch); an out-of-range target (neither in ``[0, V)`` nor
``ignore_index``) yields a NaN loss instead of an out-of-bounds read.
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


class _FwdModule:
    """Stands where the reference's JIT-built forward module stood."""

    @staticmethod
    def cross_entropy_fwd_hip(logits, targets, softcap, ignore_index, label_smoothing,
                              write_grad, save_max_sum, scale_grad):
        """Returns ``[losses, lse, row_max, row_sum, grad_logits]`` (None where not requested)."""
        _lib.require_device(logits, targets)
        if logits.dim() != 2:
            raise ValueError("logits must be [batch, vocab]")
        _lib.dtype_code(logits.dtype)
        if logits.stride(-1) != 1:
            logits = logits.contiguous()
        targets = targets.contiguous().to(torch.int64)
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
        if logits.stride(-1) != 1:
            logits = logits.contiguous()
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
    """CE with fused (gradient written in the forward) or tiny (recompute) backward.

    Arguments and return values as ``kernels/ce_fused.py:557-698`` of the
    reference: ``(logits, targets, softcap, ignore_index, label_smoothing,
    mode, return_z, z_loss_weight)`` -> loss, or ``(loss, lse)`` if return_z.
    """

    @staticmethod
    def forward(ctx, logits, targets, softcap, ignore_index, label_smoothing, mode, return_z,
                z_loss_weight=0.0):
        mod = _get_fwd_module()
        B = logits.size(0)
        z_loss_weight = float(z_loss_weight)
        if z_loss_weight > 0.0 and mode != "tiny":
            mode = "tiny"
        write_grad = 1 if mode == "fused" else 0
        save_max_sum = 1 if mode == "tiny" else 0

        if ignore_index is not None:
            valid_mask = targets != ignore_index
            n_valid_t = valid_mask.sum().to(torch.float32).clamp_(min=1.0)
        else:
            valid_mask = None
            n_valid_t = torch.tensor(float(B), device=logits.device, dtype=torch.float32)

        if write_grad:
            n_valid_scalar = n_valid_t.item()
            scale_grad = 1.0 / n_valid_scalar
        else:
            n_valid_scalar = float(B)
            scale_grad = 1.0

        ign = int(ignore_index) if ignore_index is not None else -(2 ** 63)
        losses, lse, row_max, row_sum, grad_logits = mod.cross_entropy_fwd_hip(
            logits, targets, float(softcap), ign, float(label_smoothing), int(write_grad),
            int(save_max_sum), float(scale_grad))

        if valid_mask is not None:
            loss = (losses * valid_mask.to(torch.float32)).sum() / n_valid_t
        else:
            loss = losses.mean()

        if z_loss_weight > 0.0:
            if valid_mask is not None:
                lse_valid = lse * valid_mask.to(lse.dtype)
                z_loss = z_loss_weight * (lse_valid * lse_valid).sum() / n_valid_t
            else:
                z_loss = z_loss_weight * lse.pow(2).mean()
            loss = loss + z_loss

        ctx.mode = mode
        ctx.softcap = float(softcap)
        ctx.ignore_index = ign
        ctx.has_ignore = ignore_index is not None
        ctx.label_smoothing = float(label_smoothing)
        ctx.return_z = bool(return_z)
        ctx.n_valid_item = n_valid_scalar
        ctx.n_valid_t = n_valid_t
        ctx.z_loss_weight = z_loss_weight
        if mode == "fused":
            ctx.save_for_backward(grad_logits)
            ctx.has_tiny = False
        else:
            ctx.save_for_backward(logits, targets, row_max, row_sum)
            ctx.has_tiny = True
        ctx.mark_non_differentiable(lse)
        if return_z:
            return loss, lse
        return loss

    @staticmethod
    def backward(ctx, grad_loss, *rest):
        nones = (None,) * 7
        if ctx.has_tiny:
            logits, targets, row_max, row_sum = ctx.saved_tensors
            # The loss is a mean over non-ignored rows, so its gradient is
            # scaled by 1 / n_valid (torch.nn.functional.cross_entropy's
            # gradient); the reference's tiny mode used 1 / batch here
            # (kernels/ce_fused.py:607, :661).
            n_valid = float(ctx.n_valid_t.item())
            g = float(grad_loss.item()) if grad_loss.dim() == 0 else 1.0
            grad_logits = _get_bwd_module().cross_entropy_bwd_tiny_hip(
                logits, targets, row_max, row_sum, ctx.softcap, ctx.ignore_index,
                ctx.label_smoothing, g / n_valid)
            if ctx.z_loss_weight > 0.0:
                # d/dx_ij of w * lse_i^2 / N = (2 w / N) * lse_i * softmax_ij
                with torch.no_grad():
                    shifted = logits.float() - row_max.unsqueeze(-1)
                    softmax = torch.exp(shifted) / row_sum.unsqueeze(-1)
                    lse_vec = row_max + torch.log(row_sum)
                    coef = (2.0 * ctx.z_loss_weight / n_valid) * g
                    z_grad = coef * lse_vec.unsqueeze(-1) * softmax
                    if ctx.has_ignore:
                        z_grad = z_grad * (targets != ctx.ignore_index).float().unsqueeze(-1)
                    grad_logits = grad_logits + z_grad.to(grad_logits.dtype)
            return (grad_logits,) + nones
        (saved_grad,) = ctx.saved_tensors
        if grad_loss.dim() == 0 and grad_loss.item() == 1.0:
            return (saved_grad,) + nones
        return (saved_grad * grad_loss.to(saved_grad.dtype),) + nones


def kernel_fn(logits: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    """Mean cross-entropy; matches ``reference.cross_entropy_ref`` (ignore_index -100)."""
    _lib.require_device(logits, targets)
    if not (logits.requires_grad and torch.is_grad_enabled()):
        losses, _, _, _, _ = _get_fwd_module().cross_entropy_fwd_hip(
            logits, targets, 0.0, -100, 0.0, 0, 0, 1.0)
        valid = (targets != -100).to(torch.float32)
        n_valid = valid.sum().clamp(min=1.0)
        return (losses * valid).sum() / n_valid
    return _CrossEntropyHIP.apply(logits, targets, 0.0, -100, 0.0, "fused", False, 0.0)


def ce_full(logits: torch.Tensor, targets: torch.Tensor, *, softcap: float = 0.0,
            ignore_index: int = -100, label_smoothing: float = 0.0, mode: str = "fused",
            return_z: bool = False, z_loss_weight: float = 0.0):
    """Full-featured CE; arguments as ``kernels/ce_fused.py:726-785`` of the reference."""
    _lib.require_device(logits, targets)
    if mode not in ("fused", "tiny"):
        raise ValueError(f"mode must be 'fused' or 'tiny', got {mode!r}")
    return _CrossEntropyHIP.apply(logits, targets, softcap, ignore_index, label_smoothing, mode,
                                  return_z, float(z_loss_weight))
