"""AutoKernel -- fused RMSNorm backward on gfx950 (MI355X).

Drop-in for the reference module ``kernels/hip/rmsnorm_backward.py``
(``kernel_fn`` at :239-281, kernel at :60-189). The kernel is
``ak_rmsnorm_bwd`` in ``csrc/rownorm_bwd.hip``: per row, in fp32,

    r = 1 / sqrt(mean(x^2) + eps),  n = x * r,  g = grad_output * weight
    grad_x = r * (g - n * sum(g * n) / D)
    grad_weight = sum over rows of grad_output * n        (fp32)

one read of x and grad_output, one write of grad_x; the row pass keeps each
thread's weight-gradient columns in registers and a second pass sums the
per-workgroup partial rows in a fixed order (the reference used fp32
atomics, so its grad_weight varied from run to run).

Differences from the reference, all deliberate: fp32, fp16 and bf16 run on
the kernel (the reference ran fp16 only and fell back to PyTorch otherwise);
``eps`` is a keyword (default 1e-6, the reference constant).
"""

import os

import torch

from kernels.hip import _lib

KERNEL_TYPE = "rmsnorm_backward"
BACKEND = "hip"

HIP_SRC = os.path.join(_lib.CSRC_DIR, "rownorm_bwd.hip")

DEFAULT_EPS = 1e-6


def _rows(t: torch.Tensor, d: int) -> torch.Tensor:
    return _lib.as_rows(t, d)


def kernel_fn(x: torch.Tensor, weight: torch.Tensor, grad_output: torch.Tensor,
              eps: float = DEFAULT_EPS) -> tuple:
    """Fused RMSNorm backward.

    Args:
        x: ``(..., D)`` forward input.
        weight: ``(D,)`` RMSNorm weight.
        grad_output: gradient of the RMSNorm output, shape of ``x``.

    Returns:
        ``(grad_x, grad_weight)``: grad_x with the shape and dtype of ``x``,
        grad_weight fp32 ``(D,)``.
    """
    _lib.require_device(x, weight, grad_output)
    _lib.dtype_code(x.dtype)
    D = x.shape[-1]
    if weight.dim() != 1 or weight.numel() != D:
        raise ValueError(f"weight shape {tuple(weight.shape)} does not match last dim {D}")
    if grad_output.shape != x.shape:
        raise ValueError(f"grad_output shape {tuple(grad_output.shape)} != x shape {tuple(x.shape)}")
    w = weight.to(x.dtype).contiguous()
    g = grad_output.to(x.dtype)
    x2, g2 = _rows(x, D), _rows(g, D)
    grad_x = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    grad_weight = torch.empty(D, dtype=torch.float32, device=x.device)
    ws = torch.empty(_lib.rmsnorm_bwd_workspace_bytes(x2.shape[0], D), dtype=torch.uint8,
                     device=x.device)
    _lib.rmsnorm_bwd(x2, w, g2, grad_x.view(-1, D), grad_weight, ws, eps)
    return grad_x, grad_weight
