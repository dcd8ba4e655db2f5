"""AutoKernel -- fused residual add + RMSNorm backward on gfx950 (MI355X).

Drop-in for the reference module
``kernels/hip/fused_residual_rmsnorm_backward.py`` (``kernel_fn`` at
:248-298, kernel at :61-197). Given the saved ``hidden = x + residual`` of
the dual-output forward and the gradients of both outputs, the kernel
(``ak_fused_add_rmsnorm_bwd`` in ``csrc/rownorm_bwd.hip``) computes in fp32

    r = 1 / sqrt(mean(hidden^2) + eps),  n = hidden * r,  g = grad_normed * weight
    grad_x = grad_residual = grad_hidden + r * (g - n * sum(g * n) / D)
    grad_weight = sum over rows of grad_normed * n            (fp32)

with one read of each input and one write of grad_x. ``grad_hidden`` may be
``None`` (the hidden output had no gradient). grad_weight is summed in a
fixed order (deterministic; the reference used fp32 atomics).
"""

import os
from typing import Optional

import torch

from kernels.hip import _lib

KERNEL_TYPE = "fused_residual_rmsnorm_backward"
BACKEND = "hip"

HIP_SRC = os.path.join(_lib.CSRC_DIR, "rownorm_bwd.hip")

DEFAULT_EPS = 1e-6


def _rows(t: torch.Tensor, d: int) -> torch.Tensor:
    return _lib.as_rows(t, d)


def kernel_fn(hidden: torch.Tensor, weight: torch.Tensor, grad_hidden: Optional[torch.Tensor],
              grad_normed: torch.Tensor, eps: float = DEFAULT_EPS) -> tuple:
    """Fused residual + RMSNorm backward.

    Returns ``(grad_x, grad_residual, grad_weight)``: grad_x and grad_residual
    are the same tensor (shape and dtype of ``hidden``), grad_weight is fp32.
    """
    _lib.require_device(hidden, weight, grad_hidden, grad_normed)
    _lib.dtype_code(hidden.dtype)
    D = hidden.shape[-1]
    if weight.dim() != 1 or weight.numel() != D:
        raise ValueError(f"weight shape {tuple(weight.shape)} does not match last dim {D}")
    for name, t in (("grad_hidden", grad_hidden), ("grad_normed", grad_normed)):
        if t is not None and t.shape != hidden.shape:
            raise ValueError(f"{name} shape {tuple(t.shape)} != hidden shape {tuple(hidden.shape)}")
    w = weight.to(hidden.dtype).contiguous()
    h2 = _rows(hidden, D)
    gn2 = _rows(grad_normed.to(hidden.dtype), D)
    gh2 = _rows(grad_hidden.to(hidden.dtype), D) if grad_hidden is not None else None
    grad_x = torch.empty(hidden.shape, dtype=hidden.dtype, device=hidden.device)
    grad_weight = torch.empty(D, dtype=torch.float32, device=hidden.device)
    ws = torch.empty(_lib.rmsnorm_bwd_workspace_bytes(h2.shape[0], D), dtype=torch.uint8,
                     device=hidden.device)
    _lib.fused_add_rmsnorm_bwd(h2, w, gh2, gn2, grad_x.view(-1, D), grad_weight, ws, eps)
    return grad_x, grad_x, grad_weight
