"""AutoKernel -- fused residual add + RMSNorm on gfx950 (MI355X).

Drop-in for the reference module ``kernels/hip/fused_residual_add_rmsnorm.py``
(``kernel_fn`` :340-374, ``kernel_fn_dual`` :377-418). One kernel,
``ak_fused_add_rmsnorm_fwd`` in ``csrc/rownorm.hip``, reads ``x`` and
``residual`` once, forms ``hidden = round(x + residual)`` in the input dtype,
reduces ``sum(hidden^2)`` in fp32 and writes ``hidden`` (dual variant) and
``round((hidden / rms) * weight)``: 2 reads + 2 writes per element, the HBM
minimum for the dual-output op.

Semantics follow ``reference.py:71-78``. Differences from the reference
module, all deliberate: bf16 and fp32 run on the GPU kernel instead of a
PyTorch fallback, and ``eps`` is a keyword argument (default 1e-6, the
reference's hard-coded value).
"""

import os

import torch

from kernels.hip import _lib

KERNEL_TYPE = "fused_residual_add_rmsnorm"
BACKEND = "hip"

HIP_SRC = os.path.join(_lib.CSRC_DIR, "rownorm.hip")
HIP_SRC_DUAL = HIP_SRC

DEFAULT_EPS = 1e-6


def _prepare(x, residual, weight):
    _lib.require_device(x, residual, weight)
    _lib.dtype_code(x.dtype)
    if residual.shape != x.shape:
        raise ValueError(f"residual shape {tuple(residual.shape)} != x shape {tuple(x.shape)}")
    if weight.dim() != 1 or weight.numel() != x.shape[-1]:
        raise ValueError(f"weight shape {tuple(weight.shape)} does not match last dim {x.shape[-1]}")
    if residual.dtype != x.dtype:
        residual = residual.to(x.dtype)
    if weight.dtype != x.dtype:
        weight = weight.to(x.dtype)
    n = x.shape[-1]
    x2 = _lib.as_rows(x, n)
    r2 = _lib.as_rows(residual, n)
    return x2, r2, weight.contiguous()


def kernel_fn(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
              eps: float = DEFAULT_EPS) -> torch.Tensor:
    """RMSNorm(x + residual) * weight; matches ``reference.fused_residual_add_rmsnorm_ref``."""
    x2, r2, w = _prepare(x, residual, weight)
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if y.numel():
        _lib.fused_add_rmsnorm(x2, r2, w, None, y.view(-1, x.shape[-1]), eps)
    return y


def kernel_fn_dual(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                   eps: float = DEFAULT_EPS) -> tuple:
    """Returns ``(hidden, normed)`` with ``hidden = x + residual``."""
    x2, r2, w = _prepare(x, residual, weight)
    hidden = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    normed = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if hidden.numel():
        n = x.shape[-1]
        _lib.fused_add_rmsnorm(x2, r2, w, hidden.view(-1, n), normed.view(-1, n), eps)
    return hidden, normed
