"""AutoKernel -- selective scans on gfx950 (MI355X).

Two entry points, both drop-ins:

* ``kernel_fn(dA, dBx, C, D, x)`` -- the reference's diagonal recurrence
  (``kernels/hip/selective_scan.py:214-241``)::

      state[t] = dA[t] * state[t-1] + dBx[t];   y[t] = C[t] * state[t] + D * x[t]

  over fp32 ``[batch, seq, d_inner]`` tensors (``ak_diag_scan_fwd``).

* ``selective_scan_fn(u, delta, A, B, C, D=None, z=None, delta_bias=None,
  delta_softplus=False, return_last_state=False)`` -- the Mamba-1 forward
  with the signature of ``mamba_ssm.ops.selective_scan_interface``
  (``external/mamba/mamba_ssm/ops/selective_scan_interface.py:106-112``),
  computed by ``ak_selective_scan_fwd`` with fp32 state. Results follow
  ``selective_scan_ref`` (``:115-181``) except that ``silu(z)`` is evaluated
  in fp32 rather than in ``z``'s dtype.

  Accepted layouts: ``u, delta, z`` ``[batch, dim, seqlen]`` (last dim
  contiguous), ``A`` real ``[dim, dstate]`` with ``dstate <= 256`` (the
  reference binding's limit, ``selective_scan.cpp:262``), ``B`` / ``C``
  ``[batch, dstate, seqlen]`` or ``[batch, ngroups, dstate, seqlen]``
  (input-dependent, fp32 or ``u``'s dtype) or ``[dim, dstate]``
  (input-independent, computed in fp32, as the reference's
  ``!is_variable_B`` path, ``selective_scan_interface.py:138-160``).
  ``delta`` may be fp32 or ``u``'s dtype. dstate <= 16 with input-dependent
  B / C runs the specialised kernels; everything else the general ones.
  Complex ``A`` (complex64 ``[dim, dstate]``, the reference binding's
  complex weights, ``selective_scan.cpp:236-240``) runs the complex kernels:
  an input-dependent ``B`` / ``C`` is then real ``[batch, (ngroups,) dstate,
  2 * seqlen]`` of (re, im) pairs per step, an input-independent one complex
  ``[dim, dstate]``; the state, ``last_state`` and ``dA`` are complex and
  ``out`` is ``2 Re(sum_n h C) + D u`` (``selective_scan_interface.py:
  140-145, :173-174``). The backward (``ak_selective_scan_bwd``) returns every input
  gradient of the reference's ``selective_scan_cuda.bwd``: ``du``,
  ``ddelta``, ``dA``, ``dB``, ``dC``, ``dD``, ``dz``, ``ddelta_bias``, each
  computed deterministically (fixed summation order); an input-dependent
  ``dB`` / ``dC`` is summed in fp32 and rounded once to B's / C's dtype, as
  the reference's fp32 accumulation and ``dB.to(B.dtype())``
  (``selective_scan.cpp:461``, ``:488``).

  Memory of the training path: when autograd records the call, the forward
  keeps its state every 16 steps for the backward (fp32 ``[batch,
  ceil(seqlen / 16), dim, dstate]``: 4 * dstate / 16 bytes per (batch, dim,
  step), i.e. 134 MB at batch 4, seqlen 4096, dim 2048, dstate 16, about
  twice a bf16 ``u``, and 16x that at dstate 256) plus, with a gate, its
  pre-gate output (one more ``u``-sized tensor). The reference keeps only its
  2048-step chunk states and recomputes. :func:`set_save_states` (or
  ``AUTOKERNEL_SCAN_RECOMPUTE=1`` at import) switches to recomputation;
  ``SAVE_STATES_MAX_BYTES`` caps the checkpoint size above which a call
  recomputes instead.
"""

import os

import torch

from kernels.hip import _lib

KERNEL_TYPE = "selective_scan"
BACKEND = "hip"

HIP_SRC = os.path.join(_lib.CSRC_DIR, "selective_scan.hip")

# steps per entry of the chunk-state output (the reference binding's chunk,
# external/mamba/csrc/selective_scan/selective_scan.cpp:307)
CHUNK = 2048
# Steps between the states the forward keeps for the backward (the kernels' block).
CHECKPOINT_STEPS = 16
# Training keeps those states (fp32, batch x ceil(seqlen / 16) x dim x dstate: at
# dstate 16 about twice the bytes of a bf16 u) so that the backward does not re-run
# the forward; AUTOKERNEL_SCAN_RECOMPUTE=1 (or set_save_states(False)) recomputes.
SAVE_STATES = os.environ.get("AUTOKERNEL_SCAN_RECOMPUTE", "0") != "1"
# Calls whose checkpoints would exceed this many bytes recompute instead (None: no cap).
SAVE_STATES_MAX_BYTES = None


def set_save_states(enabled: bool, max_bytes=None) -> None:
    """Whether training keeps the forward's 16-step states (see the module
    docstring for their size), and the per-call size above which it does not."""
    global SAVE_STATES, SAVE_STATES_MAX_BYTES
    SAVE_STATES = bool(enabled)
    SAVE_STATES_MAX_BYTES = max_bytes


def _checkpoint_bytes(u: torch.Tensor, A: torch.Tensor) -> int:
    batch, dim, seqlen = u.shape
    per = 8 if A.is_complex() else 4
    return per * batch * dim * A.shape[1] * ((seqlen + CHECKPOINT_STEPS - 1) // CHECKPOINT_STEPS)


def kernel_fn(dA: torch.Tensor, dBx: torch.Tensor, C: torch.Tensor, D: torch.Tensor,
              x: torch.Tensor) -> torch.Tensor:
    """Diagonal SSM scan over ``[batch, seq, d_inner]`` fp32 tensors."""
    _lib.require_device(dA, dBx, C, D, x)
    if dA.dtype != torch.float32:
        raise TypeError("dA must be float32")
    if dA.dim() != 3:
        raise ValueError("dA must be 3-D [batch, seq, d_inner]")
    shape = dA.shape
    for name, t in (("dBx", dBx), ("C", C), ("x", x)):
        if t.shape != shape:
            raise ValueError(f"{name} shape {tuple(t.shape)} != dA shape {tuple(shape)}")
    if D.numel() != shape[2]:
        raise ValueError("D must have d_inner elements")
    dA, dBx, C, x = (t.float().contiguous() for t in (dA, dBx, C, x))
    D = D.float().contiguous()
    y = torch.empty_like(dA)
    _lib.diag_scan(dA, dBx, C, D, x, y)
    return y


def _normalise(u, delta, A, B, C, D, z, delta_bias):
    """Checks shapes and brings the inputs to the layouts the kernels take:
    last dims contiguous, input-dependent B / C 4-D (fp32 or u's dtype, C in
    B's dtype when both are input-dependent), input-independent B / C
    ``[dim, dstate]`` fp32, A / D / delta_bias fp32, z in u's dtype, delta in
    fp32 or u's dtype."""
    _lib.require_device(u, delta, A, B, C, D, z, delta_bias)
    if u.dim() != 3:
        raise ValueError("u must be [batch, dim, seqlen]")
    batch, dim, seqlen = u.shape
    if u.stride(-1) != 1:
        u = u.contiguous()
    if delta.stride(-1) != 1:
        delta = delta.contiguous()
    if delta.shape != u.shape:
        raise ValueError("delta must have the shape of u")
    if A.dim() != 2 or A.shape[0] != dim:
        raise ValueError("A must be [dim, dstate]")
    dstate = A.shape[1]
    cplx = A.is_complex()

    def bc(t, name):
        if cplx:
            return _bc_complex(t, name)
        if t.dim() == 2:  # input-independent
            if tuple(t.shape) != (dim, dstate):
                raise ValueError(f"input-independent {name} must be [dim, dstate], got {tuple(t.shape)}")
            return t.float()
        if t.dim() == 3:
            t = t.unsqueeze(1)
        if t.dim() != 4 or t.shape[0] != batch or t.shape[2] != dstate or t.shape[3] != seqlen \
                or dim % t.shape[1]:
            raise ValueError(f"{name} must be [batch, ngroups, dstate, seqlen] or [dim, dstate], "
                             f"got {tuple(t.shape)}")
        if t.dtype not in (torch.float32, u.dtype):
            t = t.float()
        return t if t.stride(-1) == 1 else t.contiguous()

    def _bc_complex(t, name):
        """Complex A: input-independent complex [dim, dstate], or input-dependent
        real [batch, (ngroups,) dstate, 2 seqlen] of (re, im) pairs."""
        if t.dim() == 2:
            if tuple(t.shape) != (dim, dstate):
                raise ValueError(f"input-independent {name} must be [dim, dstate], got {tuple(t.shape)}")
            return t.to(torch.complex64)
        if t.is_complex():
            raise ValueError(f"with a complex A an input-dependent {name} is real "
                             f"[batch, ngroups, dstate, 2 * seqlen] of (re, im) pairs")
        if t.dim() == 3:
            t = t.unsqueeze(1)
        if t.dim() != 4 or t.shape[0] != batch or t.shape[2] != dstate \
                or t.shape[3] != 2 * seqlen or dim % t.shape[1]:
            raise ValueError(f"{name} must be [batch, ngroups, dstate, 2 * seqlen] or [dim, dstate] "
                             f"with a complex A, got {tuple(t.shape)}")
        if t.dtype not in (torch.float32, u.dtype):
            t = t.float()
        return t if t.stride(-1) == 1 else t.contiguous()

    B, C = bc(B, "B"), bc(C, "C")
    if B.dim() == 4 and C.dim() == 4:
        if C.shape != B.shape:
            raise ValueError(f"B / C must have one shape, got {tuple(B.shape)}, {tuple(C.shape)}")
        if C.dtype != B.dtype:
            C = C.to(B.dtype)
    A = A.to(torch.complex64) if cplx else A.float()
    if A.stride(1) != 1:
        A = A.contiguous()
    if D is not None:
        D = D.float().contiguous()
    if delta_bias is not None:
        delta_bias = delta_bias.float().contiguous()
    if z is not None:
        if z.shape != u.shape:
            raise ValueError("z must have the shape of u")
        if z.dtype != u.dtype:
            z = z.to(u.dtype)
        if z.stride(-1) != 1:
            z = z.contiguous()
    if delta.dtype not in (torch.float32, u.dtype):
        delta = delta.float()
    return u, delta, A, B, C, D, z, delta_bias


def _scan_forward(u, delta, A, B, C, D, z, delta_bias, delta_softplus, want_last_state,
                  want_prez=False, want_chunk_states=False, want_checkpoints=False):
    """With ``want_checkpoints`` the states before every 16-step block are kept
    (fp32 ``[batch, ceil(seqlen / 16), dim, dstate]``) together with the
    pre-gate output when there is a gate, for ``_scan_backward`` to restart
    from; they are returned after ``saved`` as ``(checkpoints, out_prez)``."""
    u, delta, A, B, C, D, z, delta_bias = _normalise(u, delta, A, B, C, D, z, delta_bias)
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    sdt = torch.complex64 if A.is_complex() else torch.float32  # state type
    out = torch.empty((batch, dim, seqlen), dtype=u.dtype, device=u.device)
    last_state = (torch.empty((batch, dim, dstate), dtype=sdt, device=u.device)
                  if want_last_state else None)
    prez = torch.empty_like(out) if want_prez or (want_checkpoints and z is not None) else None
    chunks = (torch.empty((batch, dim, (seqlen + CHUNK - 1) // CHUNK, dstate, 2), dtype=sdt,
                          device=u.device) if want_chunk_states else None)
    ckpt = (torch.empty((batch, (seqlen + CHECKPOINT_STEPS - 1) // CHECKPOINT_STEPS, dim, dstate),
                        dtype=sdt, device=u.device) if want_checkpoints else None)
    _lib.selective_scan(u, delta, A, B, C, D, z, delta_bias, out, last_state, delta_softplus,
                        out_prez=prez, chunk_states=chunks, checkpoints=ckpt)
    saved = (u, delta, A, B, C, D, z, delta_bias)
    if want_checkpoints:
        return out, last_state, saved, (ckpt, prez)
    if want_prez or want_chunk_states:
        return out, last_state, saved, prez, chunks
    return out, last_state, saved


def _scan_backward(dout, u, delta, A, B, C, D, z, delta_bias, delta_softplus, checkpoints=None,
                   out_prez=None):
    """Gradients of the Mamba-1 scan for the layouts ``_scan_forward`` produced
    (``ak_selective_scan_bwd``; the reference's ``selective_scan_cuda.bwd``,
    external/mamba/csrc/selective_scan/selective_scan.cpp:339-490). Given the
    forward's checkpoints (and pre-gate output), the states are not recomputed."""
    if dout.dtype != u.dtype:
        dout = dout.to(u.dtype)
    if dout.stride(-1) != 1:
        dout = dout.contiguous()
    batch, dim, seqlen = u.shape
    dev = u.device
    du = torch.empty((batch, dim, seqlen), dtype=u.dtype, device=dev)
    ddelta = torch.empty((batch, dim, seqlen), dtype=delta.dtype, device=dev)
    dA = torch.empty(A.shape, dtype=A.dtype, device=dev)
    dB = torch.empty(B.shape, dtype=B.dtype, device=dev)
    dC = torch.empty(C.shape, dtype=C.dtype, device=dev)
    dD = torch.empty(dim, dtype=torch.float32, device=dev) if D is not None else None
    dz = torch.empty((batch, dim, seqlen), dtype=u.dtype, device=dev) if z is not None else None
    dbias = torch.empty(dim, dtype=torch.float32, device=dev) if delta_bias is not None else None
    _lib.selective_scan_bwd(u, delta, A, B, C, D, z, delta_bias, dout, du, ddelta, dA, dB, dC, dD,
                            dz, dbias, delta_softplus, checkpoints=checkpoints, out_prez=out_prez)
    return du, ddelta, dA, dB, dC, dD, dz, dbias


class SelectiveScanFn(torch.autograd.Function):
    """Forward and backward on gfx950 (mirrors the reference's
    ``SelectiveScanFn``, external/mamba/mamba_ssm/ops/selective_scan_interface.py:20-83).
    When a gradient is needed the forward keeps its states every 16 steps
    (``SAVE_STATES``), so the backward does not re-run the forward; otherwise
    the backward recomputes them from the saved inputs, as the reference does."""

    @staticmethod
    def forward(ctx, u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                return_last_state=False, grad_mode=None):
        # grad_mode: whether autograd was recording at the call (forward itself
        # runs without it); needs_input_grad alone is also true under no_grad
        # for inputs that require grad, e.g. parameters during inference
        keep = (SAVE_STATES and any(ctx.needs_input_grad[:8]) and grad_mode is not False
                and (SAVE_STATES_MAX_BYTES is None
                     or _checkpoint_bytes(u, A) <= SAVE_STATES_MAX_BYTES))
        res = _scan_forward(u, delta, A, B, C, D, z, delta_bias, delta_softplus, return_last_state,
                            want_checkpoints=keep)
        out, last_state, saved = res[:3]
        ckpt, prez = res[3] if keep else (None, None)
        ctx.has_ckpt = ckpt is not None
        ctx.has_prez = prez is not None
        ctx.delta_softplus = bool(delta_softplus)
        ctx.squeeze_B = B.dim() == 3
        ctx.squeeze_C = C.dim() == 3
        ctx.bc_dtypes = (B.dtype, C.dtype)
        ctx.has_D = D is not None
        ctx.has_z = z is not None
        ctx.has_bias = delta_bias is not None
        ctx.save_for_backward(*(t for t in saved + (ckpt, prez) if t is not None))
        if return_last_state:
            ctx.mark_non_differentiable(last_state)
            return out, last_state
        return out

    @staticmethod
    def backward(ctx, dout, *args):
        it = iter(ctx.saved_tensors)
        u, delta, A, B, C = (next(it) for _ in range(5))
        D = next(it) if ctx.has_D else None
        z = next(it) if ctx.has_z else None
        delta_bias = next(it) if ctx.has_bias else None
        ckpt = next(it) if ctx.has_ckpt else None
        prez = next(it) if ctx.has_prez else None
        du, ddelta, dA, dB, dC, dD, dz, dbias = _scan_backward(
            dout, u, delta, A, B, C, D, z, delta_bias, ctx.delta_softplus, ckpt, prez)
        if ctx.squeeze_B:
            dB = dB.squeeze(1)
        if ctx.squeeze_C:
            dC = dC.squeeze(1)
        dB, dC = dB.to(ctx.bc_dtypes[0]), dC.to(ctx.bc_dtypes[1])
        return du, ddelta, dA, dB, dC, dD, dz, dbias, None, None, None


def selective_scan_fn(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                      return_last_state=False):
    """Mamba-1 selective scan. Returns ``out`` or ``(out, last_state)``."""
    return SelectiveScanFn.apply(u, delta, A, B, C, D, z, delta_bias, delta_softplus,
                                 return_last_state, torch.is_grad_enabled())
