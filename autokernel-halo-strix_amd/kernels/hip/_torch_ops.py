"""torch.library custom ops over the gfx950 kernels.

Same op names and schemas as the reference (``kernels/hip/_torch_ops.py``):

* ``autokernel::rmsnorm(Tensor x, Tensor weight, float eps=1e-6) -> Tensor``
  (:56-111)
* ``autokernel::fused_res_rmsnorm(Tensor x, Tensor residual, Tensor weight,
  float eps=1e-6) -> (Tensor, Tensor)`` (:240-303)
* ``autokernel::selective_scan(Tensor dA, Tensor dBx, Tensor C, Tensor D,
  Tensor x) -> Tensor`` (:312-394)

The trailing ``eps`` (default 1e-6, the reference's fixed value) is an
addition, so reference call sites are unchanged. Each op has ``register_fake`` (shape propagation for torch.compile) and
``register_autograd``. The forwards run the gfx950 kernels. The norm
backwards run the gfx950 backward kernels (``kernels.hip.rmsnorm_backward``,
``kernels.hip.fused_residual_rmsnorm_backward``), as the reference did for
fp16 (``_torch_ops.py:77-80``, ``:266-271``); ``AUTOKERNEL_NO_BWD_HIP=1``
selects the same gradient as fp32 PyTorch formulas on the GPU instead (the
gradient of ``rmsnorm_backward.py:166-168`` /
``fused_residual_rmsnorm_backward.py:168-170``). The diagonal scan's backward
runs ``kernels.hip.selective_scan_backward`` (the gradient of the reference's
sequential formula, ``_torch_ops.py:346-386``); its formula path is torch
autograd through the recurrence written as torch ops. Importing this module registers the ops.

Autocast: under ``torch.autocast("cuda", dtype=...)`` floating inputs are
cast to the active autocast dtype (fp16 or bf16) before the kernel runs.
The reference registered a fixed fp16 cast; following the autocast dtype
keeps fp16 behaviour identical and lets bf16 autocast reach the bf16
kernels.
"""

import os
from typing import Tuple

import torch

# Environment switch: AUTOKERNEL_NO_BWD_HIP=1 makes the backwards use the
# fp32 PyTorch formulas below instead of the gfx950 backward kernels (the
# reference's switch of the same name, _torch_ops.py:20-50).
_BWD_KERNELS_ENABLED = os.environ.get("AUTOKERNEL_NO_BWD_HIP", "0") != "1"

RMSNORM_EPS = 1e-6

_is_compiling = getattr(getattr(torch, "compiler", None), "is_compiling", None) or (lambda: False)


def _bwd_kernels_for(t: torch.Tensor) -> bool:
    """True when the backward of an op on ``t`` runs the gfx950 kernels.

    The formulas take over when the kernels are switched off and while
    torch.compile traces the backward (the formulas are traceable torch ops;
    the library calls go through ctypes and are not)."""
    return _BWD_KERNELS_ENABLED and t.is_cuda and not _is_compiling()


def disable_hip_backward():
    """Use the PyTorch formulas for every backward from now on."""
    global _BWD_KERNELS_ENABLED
    _BWD_KERNELS_ENABLED = False


def _register_autocast(op) -> None:
    """AutocastCUDA rule: cast floating CUDA inputs to the active autocast dtype."""
    keyset = (torch._C.DispatchKeySet(torch._C.DispatchKey.AutocastCPU)
              | torch._C.DispatchKeySet(torch._C.DispatchKey.AutocastCUDA))

    def kernel(_, *args):
        dt = torch.get_autocast_dtype("cuda")
        cast = tuple(a.to(dt) if isinstance(a, torch.Tensor) and a.is_floating_point() and a.is_cuda else a
                     for a in args)
        with torch._C._ExcludeDispatchKeyGuard(keyset):
            return op._opoverload(*cast)

    op._lib.impl(op._name, kernel, "AutocastCUDA", with_keyset=True)


# ---------------------------------------------------------------------------
# RMSNorm: y = x / sqrt(mean(x^2) + eps) * weight
# ---------------------------------------------------------------------------

@torch.library.custom_op("autokernel::rmsnorm", mutates_args=())
def rmsnorm_op(x: torch.Tensor, weight: torch.Tensor, eps: float = RMSNORM_EPS) -> torch.Tensor:
    from kernels.hip.rmsnorm import kernel_fn
    return kernel_fn(x, weight, eps)


@rmsnorm_op.register_fake
def _(x, weight, eps=RMSNORM_EPS):
    return x.new_empty(x.shape)


def _rmsnorm_setup(ctx, inputs, output):
    x, weight, eps = inputs
    ctx.save_for_backward(x, weight)
    ctx.eps = eps


def _rmsnorm_backward(ctx, grad_output):
    x, weight = ctx.saved_tensors
    eps = ctx.eps
    if _bwd_kernels_for(x):
        from kernels.hip.rmsnorm_backward import kernel_fn as rmsnorm_bwd_fn
        grad_x, grad_weight = rmsnorm_bwd_fn(x, weight, grad_output, eps)
        return grad_x, grad_weight.to(weight.dtype), None
    x_f = x.float()
    w_f = weight.float()
    g_f = grad_output.float()
    rms_inv = (x_f.pow(2).mean(-1, keepdim=True) + eps).rsqrt()
    normed = x_f * rms_inv
    D = x_f.shape[-1]
    grad_weight = (g_f * normed).sum(dim=tuple(range(g_f.ndim - 1)))
    grad_normed = g_f * w_f
    # d/dx of x * r * w with r = (mean(x^2) + eps)^-1/2; the projection term
    # carries one more factor of r (the reference's HIP backward kernel,
    # rmsnorm_backward.py:166-168; its PyTorch fallback, _torch_ops.py:95, drops it).
    grad_x = rms_inv * (grad_normed - normed * (grad_normed * normed).sum(-1, keepdim=True) / D)
    return grad_x.to(x.dtype), grad_weight.to(weight.dtype), None


rmsnorm_op.register_autograd(_rmsnorm_backward, setup_context=_rmsnorm_setup)
_register_autocast(rmsnorm_op)


# ---------------------------------------------------------------------------
# Fused residual add + RMSNorm: returns (hidden, normed)
# ---------------------------------------------------------------------------

@torch.library.custom_op("autokernel::fused_res_rmsnorm", mutates_args=())
def fused_res_rmsnorm_op(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                         eps: float = RMSNORM_EPS) -> Tuple[torch.Tensor, torch.Tensor]:
    from kernels.hip.fused_residual_add_rmsnorm import kernel_fn_dual
    return kernel_fn_dual(x, residual, weight, eps)


@fused_res_rmsnorm_op.register_fake
def _(x, residual, weight, eps=RMSNORM_EPS):
    return x.new_empty(x.shape), x.new_empty(x.shape)


def _fused_res_rmsnorm_setup(ctx, inputs, output):
    x, residual, weight, eps = inputs
    hidden, normed = output
    ctx.save_for_backward(hidden, weight)
    ctx.eps = eps


def _fused_res_rmsnorm_backward(ctx, grad_hidden, grad_normed):
    hidden, weight = ctx.saved_tensors
    eps = ctx.eps
    if _bwd_kernels_for(hidden) and grad_normed is not None:
        from kernels.hip.fused_residual_rmsnorm_backward import kernel_fn as fused_bwd_fn
        grad_x, _, grad_weight = fused_bwd_fn(hidden, weight, grad_hidden, grad_normed, eps)
        return grad_x, grad_x, grad_weight.to(weight.dtype), None
    if grad_normed is None:
        gx = grad_hidden.to(hidden.dtype)
        return gx, gx, torch.zeros_like(weight), None
    h_f = hidden.float()
    w_f = weight.float()
    gn_f = grad_normed.float()
    rms_inv = (h_f.pow(2).mean(-1, keepdim=True) + eps).rsqrt()
    normed_h = h_f * rms_inv
    D = h_f.shape[-1]
    grad_weight = (gn_f * normed_h).sum(dim=tuple(range(gn_f.ndim - 1)))
    gns = gn_f * w_f
    # as fused_residual_rmsnorm_backward.py:168-170 of the reference
    grad_h_from_norm = rms_inv * (gns - normed_h * (gns * normed_h).sum(-1, keepdim=True) / D)
    total = grad_h_from_norm if grad_hidden is None else grad_hidden.float() + grad_h_from_norm
    grad_x = total.to(hidden.dtype)
    return grad_x, grad_x, grad_weight.to(weight.dtype), None


fused_res_rmsnorm_op.register_autograd(_fused_res_rmsnorm_backward,
                                       setup_context=_fused_res_rmsnorm_setup)
_register_autocast(fused_res_rmsnorm_op)


# ---------------------------------------------------------------------------
# Diagonal selective scan:
#   state[t] = dA[t] * state[t-1] + dBx[t];  y[t] = C[t] * state[t] + D * x[t]
# ---------------------------------------------------------------------------

@torch.library.custom_op("autokernel::selective_scan", mutates_args=())
def selective_scan_op(dA: torch.Tensor, dBx: torch.Tensor, C: torch.Tensor, D: torch.Tensor,
                      x: torch.Tensor) -> torch.Tensor:
    from kernels.hip.selective_scan import kernel_fn
    return kernel_fn(dA, dBx, C, D, x)


@selective_scan_op.register_fake
def _(dA, dBx, C, D, x):
    return dA.new_empty(dA.shape)


def _selective_scan_setup(ctx, inputs, output):
    dA, dBx, C, D, x = inputs
    ctx.save_for_backward(dA, dBx, C, D, x, output)


def _diag_recurrence(dA, dBx, C, D, x):
    """The forward recurrence as torch ops over [batch, seq, d_inner] (a
    traceable stand-in for the kernel; its autograd gives the formula path's
    gradients)."""
    state = torch.zeros_like(dA[:, 0])
    ys = []
    for t in range(dA.shape[1]):
        state = torch.addcmul(dBx[:, t], dA[:, t], state)
        ys.append(C[:, t] * state)
    return torch.stack(ys, dim=1) + D * x


def _selective_scan_backward(ctx, grad_y):
    dA, dBx, C, D, x, _ = ctx.saved_tensors
    inputs = (dA, dBx, C, D, x)
    if _bwd_kernels_for(dA):
        # ak_diag_scan_bwd over fp32 copies (the kernel's state is fp32)
        from kernels.hip.selective_scan_backward import kernel_fn as scan_bwd_fn
        grads = scan_bwd_fn(*(t.float() for t in inputs), grad_y.float())
    else:
        with torch.enable_grad():
            leaves = [t.detach().float().requires_grad_() for t in inputs]
            y = _diag_recurrence(*leaves)
            grads = torch.autograd.grad(y, leaves, grad_y.float())
    return tuple(g.to(t.dtype) for g, t in zip(grads, inputs))


selective_scan_op.register_autograd(_selective_scan_backward, setup_context=_selective_scan_setup)
