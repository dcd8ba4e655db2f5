"""AutoKernel -- backward of the diagonal selective scan on gfx950 (MI355X).

Drop-in for the reference module ``kernels/hip/selective_scan_backward.py``
(``kernel_fn`` at :393-421). For the forward recurrence of
``kernels.hip.selective_scan.kernel_fn``

    state[t] = dA[t] * state[t-1] + dBx[t];   y[t] = C[t] * state[t] + D * x[t]

the kernel (``ak_diag_scan_bwd`` in ``csrc/selective_scan.hip``) recomputes
the states forward in time into the grad_C buffer and then runs the
gradient recurrence backward in time, one lane per (batch, channel):

    grad_C[t] = gy[t] * state[t];  g += gy[t] * C[t];  grad_dA[t] = g * state[t-1]
    grad_dBx[t] = g;  g *= dA[t];  grad_x = gy * D;  grad_D = sum_{b,t} gy * x

which is the reference's sequential formula (``_torch_ops.py:346-386``);
grad_D is reduced over the batch in a fixed order.
"""

import os

import torch

from kernels.hip import _lib

KERNEL_TYPE = "selective_scan_backward"
BACKEND = "hip"

HIP_SRC = os.path.join(_lib.CSRC_DIR, "selective_scan.hip")


def kernel_fn(dA: torch.Tensor, dBx: torch.Tensor, C: torch.Tensor, D: torch.Tensor,
              x: torch.Tensor, grad_y: torch.Tensor) -> tuple:
    """Backward of the diagonal scan. All inputs fp32; ``dA``, ``dBx``, ``C``,
    ``x``, ``grad_y`` ``[batch, seq, d_inner]``, ``D`` ``[d_inner]``.

    Returns ``(grad_dA, grad_dBx, grad_C, grad_D, grad_x)``, all fp32.
    """
    _lib.require_device(dA, dBx, C, D, x, grad_y)
    if dA.dtype != torch.float32:
        raise TypeError("dA must be float32")
    if dA.dim() != 3:
        raise ValueError("dA must be 3-D [batch, seq, d_inner]")
    shape = dA.shape
    for name, t in (("dBx", dBx), ("C", C), ("x", x), ("grad_y", grad_y)):
        if t.shape != shape:
            raise ValueError(f"{name} shape {tuple(t.shape)} != dA shape {tuple(shape)}")
    if D.numel() != shape[2]:
        raise ValueError("D must have d_inner elements")
    dA, dBx, C, x, gy = (t.float().contiguous() for t in (dA, dBx, C, x, grad_y))
    D = D.float().contiguous()
    grad_dA, grad_dBx, grad_C, grad_x = (torch.empty_like(dA) for _ in range(4))
    grad_D = torch.empty(shape[2], dtype=torch.float32, device=dA.device)
    _lib.diag_scan_bwd(dA, dBx, C, D, x, gy, grad_dA, grad_dBx, grad_C, grad_D, grad_x)
    return grad_dA, grad_dBx, grad_C, grad_D, grad_x
