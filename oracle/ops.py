"""CPU oracle: restatements of the reference's arithmetic for the gfx950 kernels.

TEST INFRASTRUCTURE ONLY. Nothing in the product (the package under
``autokernel-halo-strix_amd/``) imports this module; only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use
it, as the checker / CPU baseline, never as the thing measured or shipped.

Every function restates one reference function (torch on the CPU, fp32
unless stated) and cites the reference file:line it follows. Each is pinned
by tests in ``tests/test_oracle.py`` against closed forms, invariants,
float64 brute force on tiny inputs and the reference's own known-answer test
(``scripts/test_griffin_scan_op.py:42-52``).
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

# ---------------------------------------------------------------------------
# Norms
# ---------------------------------------------------------------------------


def rmsnorm_ref(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``reference.py:25-29`` verbatim semantics: arithmetic in ``x``'s dtype."""
    rms = torch.sqrt(torch.mean(x ** 2, dim=-1, keepdim=True) + eps)
    return (x / rms) * weight


def rmsnorm_f32_ref(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm computed in fp32 and rounded once to ``x.dtype``.

    The fp32 path of ``reference.py:71-78`` applied without the residual; this
    is what the gfx950 kernel computes for fp16 / bf16 inputs (for fp32 inputs
    it equals :func:`rmsnorm_ref`).
    """
    xf = x.float()
    rms = torch.sqrt(torch.mean(xf ** 2, dim=-1, keepdim=True) + eps)
    return ((xf / rms) * weight.float()).to(x.dtype)


def fused_residual_add_rmsnorm_ref(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                                   eps: float = 1e-6) -> Tuple[torch.Tensor, torch.Tensor]:
    """``reference.py:71-78`` plus the ``hidden`` output of ``kernel_fn_dual``.

    hidden = x + residual in the input dtype (one rounding of the exact sum);
    y = ((hidden_f / sqrt(mean(hidden_f^2) + eps)) * weight_f).to(dtype).
    """
    hidden = x + residual
    hf = hidden.float()
    rms = torch.sqrt(torch.mean(hf ** 2, dim=-1, keepdim=True) + eps)
    return hidden, ((hf / rms) * weight.float()).to(x.dtype)


def rmsnorm_bwd_ref(x: torch.Tensor, weight: torch.Tensor, grad_out: torch.Tensor,
                    eps: float = 1e-6) -> Tuple[torch.Tensor, torch.Tensor]:
    """RMSNorm backward in float64 (unrounded), the gradient of
    ``kernels/hip/rmsnorm_backward.py:60-189`` (formula at :166-168):

        r = 1 / sqrt(mean(x^2) + eps), n = x * r, g = grad_out * weight
        grad_x = r * (g - n * sum(g * n) / D),  grad_weight = sum_rows(grad_out * n)

    Returns ``(grad_x, grad_weight)`` as float64 with ``x``'s shape and ``(D,)``.
    """
    xd, wd, gd = x.double(), weight.double(), grad_out.double()
    r = 1.0 / torch.sqrt(torch.mean(xd * xd, dim=-1, keepdim=True) + eps)
    n = xd * r
    g = gd * wd
    D = x.shape[-1]
    grad_x = r * (g - n * (g * n).sum(-1, keepdim=True) / D)
    grad_w = (gd * n).reshape(-1, D).sum(0)
    return grad_x, grad_w


def fused_residual_rmsnorm_bwd_ref(hidden: torch.Tensor, weight: torch.Tensor,
                                   grad_hidden: Optional[torch.Tensor], grad_normed: torch.Tensor,
                                   eps: float = 1e-6) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused residual + RMSNorm backward in float64 (unrounded), following
    ``kernels/hip/fused_residual_rmsnorm_backward.py:61-197`` (:168-178):
    grad_x = grad_residual = grad_hidden + RMSNorm-backward(hidden, grad_normed).
    Returns ``(grad_x, grad_weight)``."""
    gx, gw = rmsnorm_bwd_ref(hidden, weight, grad_normed, eps)
    if grad_hidden is not None:
        gx = gx + grad_hidden.double()
    return gx, gw


# ---------------------------------------------------------------------------
# Softmax
# ---------------------------------------------------------------------------


def softmax_ref(x: torch.Tensor) -> torch.Tensor:
    """``reference.py:14-17`` (``F.softmax(x, -1)``) with fp32 accumulation."""
    return F.softmax(x.float(), dim=-1).to(x.dtype)


# ---------------------------------------------------------------------------
# Cross-entropy over materialised logits (kernels/ce_fused.py)
# ---------------------------------------------------------------------------


def _capped(logits: torch.Tensor, softcap: float) -> torch.Tensor:
    x = logits if logits.dtype == torch.float64 else logits.float()
    if softcap > 0:
        x = softcap * torch.tanh(x / softcap)
    return x


def ce_rows_ref(logits: torch.Tensor, targets: torch.Tensor, softcap: float = 0.0,
                ignore_index: int = -100, label_smoothing: float = 0.0):
    """Per-row ``(losses, lse, row_max, row_sum)`` of ``kernels/ce_fused.py:144-262``.

    lse = max + log(sum(exp(x - max))) over the (softcapped) row; loss =
    lse - x[t], or lse - (1-a) x[t] - a mean(x) with label smoothing a;
    ignored rows: loss 0, lse still reported.
    """
    x = _capped(logits, softcap)
    row_max = x.max(dim=-1).values
    row_sum = torch.exp(x - row_max[:, None]).sum(-1)
    lse = row_max + torch.log(row_sum)
    t = targets.long()
    ignored = t == ignore_index
    tc = torch.where(ignored, torch.zeros_like(t), t)
    xt = x.gather(1, tc[:, None]).squeeze(1)
    if label_smoothing > 0:
        loss = lse - (1 - label_smoothing) * xt - label_smoothing * x.mean(-1)
    else:
        loss = lse - xt
    loss = torch.where(ignored, torch.zeros_like(loss), loss)
    return loss, lse, row_max, row_sum


def ce_grad_ref(logits: torch.Tensor, targets: torch.Tensor, softcap: float = 0.0,
                ignore_index: int = -100, label_smoothing: float = 0.0,
                scale: float = 1.0, z_loss_weight: float = 0.0) -> torch.Tensor:
    """Gradient rows of ``kernels/ce_fused.py:268-328`` (fp32).

    g = softmax(x) - [i == t](1 - a) - a / V, plus 2 w lse softmax(x) for a
    z-loss weight w (the gradient of w * lse^2, ``ce_fused.py:668-684``),
    times (1 - tanh^2) under the softcap, times ``scale``; ignored rows are
    zero.
    """
    x = _capped(logits, softcap)
    V = x.shape[-1]
    p = torch.softmax(x, dim=-1)
    if z_loss_weight > 0:
        p = p * (1 + 2 * z_loss_weight * torch.logsumexp(x, dim=-1, keepdim=True))
    t = targets.long()
    ignored = t == ignore_index
    tc = torch.where(ignored, torch.zeros_like(t), t)
    onehot = F.one_hot(tc, V).float()
    g = p - onehot * (1 - label_smoothing)
    if label_smoothing > 0:
        g = g - label_smoothing / V
    if softcap > 0:
        th = x / softcap
        g = g * (1 - th * th)
    g = g * scale
    return torch.where(ignored[:, None], torch.zeros_like(g), g)


def ce_mean_ref(losses: torch.Tensor, targets: torch.Tensor, ignore_index: int = -100,
                lse: torch.Tensor = None, z_loss_weight: float = 0.0) -> torch.Tensor:
    """Mean over non-ignored rows, denominator clamped to 1 (``ce_fused.py:594-622``),
    plus ``z_loss_weight * sum(lse^2)`` over the same rows and denominator
    (``:611-626``)."""
    ct = losses.dtype if losses.dtype == torch.float64 else torch.float32
    valid = (targets != ignore_index).to(ct)
    total = (losses * valid).sum()
    if z_loss_weight > 0:
        total = total + z_loss_weight * (lse.to(ct) ** 2 * valid).sum()
    return total / valid.sum().clamp(min=1.0)


def lmhead_ce_ref(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                  ignore_index: int = -100, vocab_chunk: int = 4096, softcap: float = 0.0,
                  label_smoothing: float = 0.0, dtype: torch.dtype = torch.float32):
    """Linear + CE without materialising all logits (``dtype`` arithmetic,
    fp32 by default, float64 for the full-size checks).

    Follows ``kernels/hip/chunked_linear_cross_entropy.py:72-75`` (n_valid),
    ``:135-140`` (loss = sum / n_valid) and ``kernels/ce_fused.py:236-260``
    (per-row loss, logit softcap ``softcap * tanh(z / softcap)`` when
    ``softcap > 0``, label smoothing a: ``lse - (1 - a) z_t - a mean(z)``,
    ``:250-256``), streaming the vocabulary in ``vocab_chunk`` columns with
    an online (max, sum) merge. Returns ``(loss, lse, losses)``.
    """
    h = hidden.to(dtype)
    V = weight.shape[0]
    n = h.shape[0]
    m = torch.full((n,), -math.inf, dtype=dtype)
    s = torch.zeros(n, dtype=dtype)
    t = targets.long()
    xt = torch.zeros(n, dtype=dtype)
    zsum = torch.zeros(n, dtype=dtype)
    for v0 in range(0, V, vocab_chunk):
        v1 = min(V, v0 + vocab_chunk)
        logits = _capped(h @ weight[v0:v1].to(dtype).t(), softcap)
        cm = logits.max(dim=-1).values
        nm = torch.maximum(m, cm)
        s = s * torch.exp(m - nm) + torch.exp(logits - nm[:, None]).sum(-1)
        m = nm
        zsum += logits.sum(-1)
        inside = (t >= v0) & (t < v1)
        if inside.any():
            idx = inside.nonzero().squeeze(1)
            xt[idx] = logits[idx, t[idx] - v0]
    lse = m + torch.log(s)
    ignored = t == ignore_index
    if label_smoothing > 0:
        per = lse - (1 - label_smoothing) * xt - label_smoothing * zsum / V
    else:
        per = lse - xt
    losses = torch.where(ignored, torch.zeros_like(lse), per)
    return ce_mean_ref(losses, t, ignore_index), lse, losses


# ---------------------------------------------------------------------------
# Scans
# ---------------------------------------------------------------------------


def _bc_per_channel(t: torch.Tensor, batch: int, dim: int, seqlen: int) -> torch.Tensor:
    """B or C as ``[batch, dim, dstate, seqlen]``: an input-dependent one
    (``[b, n, l]`` or ``[b, g, n, l]``) repeated over each group's channels, an
    input-independent one (``[dim, n]``, ``selective_scan_interface.py:
    151-152``) repeated over batch and steps."""
    if t.dim() == 2:
        return t[None, :, :, None].expand(batch, dim, t.shape[1], seqlen)
    if t.dim() == 3:
        t = t.unsqueeze(1)
    return t.repeat_interleave(dim // t.shape[1], dim=1)


def selective_scan_ref(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                       return_last_state=False, initial_state: Optional[torch.Tensor] = None,
                       silu_fp32: bool = True, compute_dtype: torch.dtype = torch.float32):
    """``external/mamba/mamba_ssm/ops/selective_scan_interface.py:115-181`` (real A).

    fp32 state; B / C given as [b, n, l] or [b, g, n, l] (groups repeated over
    dim) or input-independent [dim, n]. ``silu_fp32=True`` evaluates silu(z) in fp32 (the gfx950 kernel's
    choice); ``False`` evaluates it in z's dtype as the reference does (:179).
    ``initial_state`` [b, d, n] (fp32) starts the recurrence from a given
    state; the reference starts from zeros. ``compute_dtype=torch.float64``
    runs every step in float64 and returns float64 (for autograd checks of
    the backward).
    """
    cd = compute_dtype
    dtype_in = u.dtype if cd == torch.float32 else cd
    u = u.to(cd)
    delta = delta.to(cd)
    if delta_bias is not None:
        delta = delta + delta_bias[..., None].to(cd)
    if delta_softplus:
        delta = F.softplus(delta)
    batch, dim, dstate = u.shape[0], A.shape[0], A.shape[1]
    Bf = _bc_per_channel(B.to(cd), batch, dim, u.shape[2])  # [b, d, n, l]
    Cf = _bc_per_channel(C.to(cd), batch, dim, u.shape[2])
    x = (torch.zeros(batch, dim, dstate, dtype=cd) if initial_state is None
         else initial_state.to(cd).clone())
    deltaA = torch.exp(delta[:, :, :, None] * A.to(cd)[None, :, None, :])         # [b, d, l, n]
    deltaB_u = (delta * u)[:, :, :, None] * Bf.permute(0, 1, 3, 2)                 # [b, d, l, n]
    Cl = Cf.permute(0, 1, 3, 2)                                                   # [b, d, l, n]
    ys = []
    for i in range(u.shape[2]):
        x = deltaA[:, :, i] * x + deltaB_u[:, :, i]
        ys.append((x * Cl[:, :, i]).sum(-1))
    y = torch.stack(ys, dim=2)
    out = y if D is None else y + u * D.to(cd)[:, None]
    if z is not None:
        gate = F.silu(z.to(cd)) if (silu_fp32 or cd != torch.float32) else F.silu(z).float()
        out = out * gate
    out = out.to(dtype_in)
    return (out, x) if return_last_state else out


def selective_scan_chunk_states_ref(u, delta, A, B, delta_bias=None, delta_softplus=False,
                                    chunk: int = 2048):
    """The chunk-state output ``x`` of the reference's forward binding
    (``selective_scan.cpp:307-313``; written at
    ``selective_scan_fwd_kernel.cuh:241-258``): for every 2048-step chunk,
    the running prefix of the scan from step 0 to the chunk's last step, the
    pair (prod_s exp(delta'_s A), h) per state. float64, shape
    ``[batch, dim, n_chunks, dstate, 2]`` (the reference's ``[batch, dim,
    n_chunks, 2 * dstate]`` with interleaved pairs)."""
    f = torch.float64
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    draw = delta.to(f) + (delta_bias.to(f)[..., None] if delta_bias is not None else 0.0)
    dl = F.softplus(draw) if delta_softplus else draw
    Bd = _bc_per_channel(B.to(f), batch, dim, seqlen)  # [b, d, n, l]
    nch = (seqlen + chunk - 1) // chunk
    out = torch.empty(batch, dim, nch, dstate, 2, dtype=f)
    prod = torch.ones(batch, dim, dstate, dtype=f)
    h = torch.zeros(batch, dim, dstate, dtype=f)
    for l in range(seqlen):
        a = torch.exp(dl[:, :, l, None] * A.to(f)[None])
        prod = prod * a
        h = a * h + (dl[:, :, l] * u[:, :, l].to(f))[..., None] * Bd[..., l]
        if (l + 1) % chunk == 0 or l + 1 == seqlen:
            out[:, :, l // chunk, :, 0] = prod
            out[:, :, l // chunk, :, 1] = h
    return out


def selective_scan_bwd_ref(u, delta, A, B, C, dout, D=None, z=None, delta_bias=None,
                           delta_softplus=False):
    """Gradients of :func:`selective_scan_ref` (real A; B / C input-dependent or
    input-independent [dim, n], whose gradients sum over batch and steps), in
    float64, by the reverse recurrence of the reference's backward kernel
    (``external/mamba/csrc/selective_scan/selective_scan_bwd_kernel.cuh``:
    dz and the gated dout :189-197, dD :219, the per-step terms :284-300,
    the softplus derivative :452-455). With delta' = softplus?(delta + bias),
    a_l = exp(delta'_l A), g_l the gradient of the state after step l:

        g_l       = a_{l+1} g_{l+1} + dy_l C_l          (dy = dout * silu(z))
        du_l      = D dy_l + sum_n g_l delta'_l B_l
        ddelta'_l = sum_n g_l (u_l B_l + A a_l h_{l-1})
        dA       += g_l delta'_l a_l h_{l-1};  dB_l += g_l delta'_l u_l;  dC_l += dy_l h_l

    Returns ``(du, ddelta, dA, dB, dC, dD, dz, ddelta_bias)`` as float64
    tensors (``dB`` / ``dC`` in B's / C's layout; None for absent inputs).
    """
    f = torch.float64
    u64, dout64 = u.to(f), dout.to(f)
    draw = delta.to(f) + (delta_bias.to(f)[..., None] if delta_bias is not None else 0.0)
    dl = F.softplus(draw) if delta_softplus else draw
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    A64 = A.to(f)
    Bd = _bc_per_channel(B.to(f), batch, dim, seqlen)  # [b, d, n, l]
    Cd = _bc_per_channel(C.to(f), batch, dim, seqlen)
    a = torch.exp(dl[:, :, None, :] * A64[None, :, :, None])  # [b, d, n, l]
    x = (dl * u64)[:, :, None, :] * Bd
    h = torch.empty(batch, dim, dstate, seqlen, dtype=f)
    s = torch.zeros(batch, dim, dstate, dtype=f)
    for l in range(seqlen):
        s = a[..., l] * s + x[..., l]
        h[..., l] = s
    y = (h * Cd).sum(2)
    if D is not None:
        y = y + u64 * D.to(f)[:, None]
    if z is not None:
        z64 = z.to(f)
        sg = torch.sigmoid(z64)
        dz = dout64 * y * sg * (1 + z64 * (1 - sg))
        dy = dout64 * z64 * sg
    else:
        dz, dy = None, dout64
    g = torch.zeros(batch, dim, dstate, dtype=f)
    gh = torch.empty_like(h)
    for l in range(seqlen - 1, -1, -1):
        if l + 1 < seqlen:
            g = g * a[..., l + 1]
        g = g + dy[:, :, None, l] * Cd[..., l]
        gh[..., l] = g
    hprev = torch.cat([torch.zeros_like(h[..., :1]), h[..., :-1]], dim=-1)
    ah = a * hprev
    du = (gh * dl[:, :, None] * Bd).sum(2)
    if D is not None:
        du = du + dy * D.to(f)[:, None]
    ddl = (gh * (u64[:, :, None] * Bd + A64[None, :, :, None] * ah)).sum(2)
    dA = (gh * dl[:, :, None] * ah).sum((0, 3))
    dB_d = gh * (dl * u64)[:, :, None]  # [b, d, n, l]
    dC_d = dy[:, :, None] * h

    def fold(g_d, like):
        """The per-channel gradient back to the layout of B / C: summed over
        each group's channels, or over batch and steps for [dim, n]."""
        if like.dim() == 2:
            return g_d.sum((0, 3))
        ng = 1 if like.dim() == 3 else like.shape[1]
        out = g_d.reshape(batch, ng, dim // ng, dstate, seqlen).sum(2)
        return out.squeeze(1) if like.dim() == 3 else out

    dB, dC = fold(dB_d, B), fold(dC_d, C)
    if delta_softplus:
        ddelta = torch.where(draw <= 20.0, ddl * torch.sigmoid(draw), ddl)
    else:
        ddelta = ddl
    dD = (dy * u64).sum((0, 2)) if D is not None else None
    dbias = ddelta.sum((0, 2)) if delta_bias is not None else None
    return du, ddelta, dA, dB, dC, dD, dz, dbias


def _bc_complex(t: torch.Tensor, batch: int, dim: int, seqlen: int) -> torch.Tensor:
    """B or C of a complex-A scan as complex128 ``[batch, dim, dstate, seqlen]``.

    An input-dependent one is a real ``[b, n, 2l]`` or ``[b, g, n, 2l]`` tensor
    whose last dimension holds (re, im) pairs per step, read with
    ``view_as_complex`` (``selective_scan_interface.py:140-145``) and repeated
    over each group's channels; an input-independent one is complex
    ``[dim, n]``, repeated over batch and steps."""
    if t.is_complex():
        return t.to(torch.complex128)[None, :, :, None].expand(batch, dim, t.shape[1], seqlen)
    t = t.to(torch.float64)
    if t.dim() == 3:
        t = t.unsqueeze(1)
    tc = torch.view_as_complex(t.reshape(*t.shape[:-1], seqlen, 2).contiguous())
    return tc.repeat_interleave(dim // tc.shape[1], dim=1)


def _dl64(delta, delta_bias, delta_softplus):
    f = torch.float64
    draw = delta.to(f) + (delta_bias.to(f)[..., None] if delta_bias is not None else 0.0)
    return draw, (F.softplus(draw) if delta_softplus else draw)


def selective_scan_complex_ref(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                               delta_softplus=False, return_last_state=False):
    """``external/mamba/mamba_ssm/ops/selective_scan_interface.py:115-181`` with
    complex ``A`` (``:140-145``, ``:173-174``), in complex128 / float64.

    The state is complex; each step's output is twice the real part of
    sum_n h_n C_n (``y.real * 2``), then ``+ D u`` and the gate ``silu(z)``.
    Returns float64 ``out`` (and the complex128 last state)."""
    f, c = torch.float64, torch.complex128
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    u64 = u.to(f)
    _, dl = _dl64(delta, delta_bias, delta_softplus)
    Bd = _bc_complex(B, batch, dim, seqlen)
    Cd = _bc_complex(C, batch, dim, seqlen)
    A128 = A.to(c)
    x = torch.zeros(batch, dim, dstate, dtype=c)
    ys = []
    for l in range(seqlen):
        a = torch.exp(dl[:, :, l, None] * A128[None])
        x = a * x + (dl[:, :, l] * u64[:, :, l])[..., None] * Bd[..., l]
        ys.append(2.0 * (x * Cd[..., l]).sum(-1).real)
    y = torch.stack(ys, dim=2) if seqlen else torch.zeros(batch, dim, 0, dtype=f)
    out = y if D is None else y + u64 * D.to(f)[:, None]
    if z is not None:
        out = out * F.silu(z.to(f))
    return (out, x) if return_last_state else out


def selective_scan_complex_chunk_states_ref(u, delta, A, B, delta_bias=None, delta_softplus=False,
                                            chunk: int = 2048):
    """The chunk-state output ``x`` of the reference's forward binding for
    complex ``A`` (``selective_scan.cpp:307-313``: ``[batch, dim, n_chunks,
    2 * dstate]`` complex): per 2048-step chunk, the running prefix from step
    0 to the chunk's last step, (prod_s exp(delta'_s A), h) per state.
    complex128 ``[batch, dim, n_chunks, dstate, 2]``."""
    f, c = torch.float64, torch.complex128
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    _, dl = _dl64(delta, delta_bias, delta_softplus)
    Bd = _bc_complex(B, batch, dim, seqlen)
    nch = (seqlen + chunk - 1) // chunk
    out = torch.empty(batch, dim, nch, dstate, 2, dtype=c)
    prod = torch.ones(batch, dim, dstate, dtype=c)
    h = torch.zeros(batch, dim, dstate, dtype=c)
    for l in range(seqlen):
        a = torch.exp(dl[:, :, l, None] * A.to(c)[None])
        prod = prod * a
        h = a * h + (dl[:, :, l] * u[:, :, l].to(f))[..., None] * Bd[..., l]
        if (l + 1) % chunk == 0 or l + 1 == seqlen:
            out[:, :, l // chunk, :, 0] = prod
            out[:, :, l // chunk, :, 1] = h
    return out


def selective_scan_complex_bwd_ref(u, delta, A, B, C, dout, D=None, z=None, delta_bias=None,
                                   delta_softplus=False):
    """Gradients of :func:`selective_scan_complex_ref` by the reverse
    recurrence in complex128. A complex input's gradient is packed as
    dL/dRe + i dL/dIm (the convention of torch autograd, which the reference's
    tests compare the binding's complex ``dA`` with); for a complex z' = w z
    the packed gradient of z is conj(w) times that of z'. With a_l =
    exp(delta'_l A), h_l = a_l h_{l-1} + delta'_l u_l B_l and
    y_l = 2 Re sum_n h_l C_l:

        g_l       = conj(a_{l+1}) g_{l+1} + 2 dy_l conj(C_l)
        du_l      = D dy_l + sum_n Re(conj(g_l) delta'_l B_l)
        ddelta'_l = sum_n Re(conj(g_l) u_l B_l) + Re(conj(g_l conj(h_{l-1})) A a_l)
        dA       += delta'_l conj(a_l) g_l conj(h_{l-1})
        dB_l      = delta'_l u_l g_l;   dC_l = 2 dy_l conj(h_l)

    Returns ``(du, ddelta, dA, dB, dC, dD, dz, ddelta_bias)``: float64 except
    dA (complex128) and an input-independent dB / dC (complex128 ``[dim, n]``);
    an input-dependent dB / dC is float64 in B's / C's real interleaved layout.
    """
    f, c = torch.float64, torch.complex128
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    u64, dout64 = u.to(f), dout.to(f)
    draw, dl = _dl64(delta, delta_bias, delta_softplus)
    A128 = A.to(c)
    Bd = _bc_complex(B, batch, dim, seqlen)
    Cd = _bc_complex(C, batch, dim, seqlen)
    a = torch.exp(dl[:, :, None, :] * A128[None, :, :, None])  # [b, d, n, l]
    bx = (dl * u64)[:, :, None, :] * Bd
    h = torch.empty(batch, dim, dstate, seqlen, dtype=c)
    s = torch.zeros(batch, dim, dstate, dtype=c)
    for l in range(seqlen):
        s = a[..., l] * s + bx[..., l]
        h[..., l] = s
    y = 2.0 * (h * Cd).sum(2).real
    if D is not None:
        y = y + u64 * D.to(f)[:, None]
    if z is not None:
        z64 = z.to(f)
        sg = torch.sigmoid(z64)
        dz = dout64 * y * sg * (1 + z64 * (1 - sg))
        dy = dout64 * z64 * sg
    else:
        dz, dy = None, dout64
    g = torch.zeros(batch, dim, dstate, dtype=c)
    gh = torch.empty_like(h)
    for l in range(seqlen - 1, -1, -1):
        if l + 1 < seqlen:
            g = g * a[..., l + 1].conj()
        g = g + 2.0 * dy[:, :, None, l] * Cd[..., l].conj()
        gh[..., l] = g
    hprev = torch.cat([torch.zeros_like(h[..., :1]), h[..., :-1]], dim=-1)
    ga = gh * hprev.conj()                                   # packed gradient of a_l
    du = (gh.conj() * dl[:, :, None] * Bd).real.sum(2)
    if D is not None:
        du = du + dy * D.to(f)[:, None]
    ddl = ((gh.conj() * u64[:, :, None] * Bd).real
           + (ga.conj() * A128[None, :, :, None] * a).real).sum(2)
    dA = (dl[:, :, None] * a.conj() * ga).sum((0, 3))
    dB_d = gh * (dl * u64)[:, :, None]
    dC_d = 2.0 * dy[:, :, None] * h.conj()

    def fold(g_d, like):
        if like.is_complex():  # input-independent [dim, n]
            return g_d.sum((0, 3))
        ng = 1 if like.dim() == 3 else like.shape[1]
        out = g_d.reshape(batch, ng, dim // ng, dstate, seqlen).sum(2)
        out = torch.view_as_real(out).reshape(batch, ng, dstate, 2 * seqlen)
        return out.squeeze(1) if like.dim() == 3 else out

    dB, dC = fold(dB_d, B), fold(dC_d, C)
    if delta_softplus:
        ddelta = torch.where(draw <= 20.0, ddl * torch.sigmoid(draw), ddl)
    else:
        ddelta = ddl
    dD = (dy * u64).sum((0, 2)) if D is not None else None
    dbias = ddelta.sum((0, 2)) if delta_bias is not None else None
    return du, ddelta, dA, dB, dC, dD, dz, dbias


def diag_scan_ref(dA, dBx, C, D, x):
    """Diagonal recurrence of ``kernels/hip/selective_scan.py:1-20, :214-241``.

    state[t] = dA[t] * state[t-1] + dBx[t];  y[t] = C[t] * state[t] + D * x[t]
    over fp32 [batch, seq, d_inner].
    """
    dA, dBx, C, x = (t.float() for t in (dA, dBx, C, x))
    batch, seqlen, d = dA.shape
    s = torch.zeros(batch, d)
    ys = []
    for t in range(seqlen):
        s = dA[:, t] * s + dBx[:, t]
        ys.append(C[:, t] * s + D.float() * x[:, t])
    return torch.stack(ys, dim=1)


def diag_scan_bwd_ref(dA, dBx, C, D, x, grad_y):
    """Backward of :func:`diag_scan_ref`, the sequential formula of
    ``kernels/hip/_torch_ops.py:346-386`` (float64). Returns
    ``(grad_dA, grad_dBx, grad_C, grad_D, grad_x)``."""
    dA, dBx, C, x, gy = (t.double() for t in (dA, dBx, C, x, grad_y))
    Dd = D.double()
    batch, seqlen, d = dA.shape
    states = torch.zeros(batch, seqlen + 1, d, dtype=torch.float64)
    for t in range(seqlen):
        states[:, t + 1] = dA[:, t] * states[:, t] + dBx[:, t]
    g_dA, g_dBx, g_C = torch.zeros_like(dA), torch.zeros_like(dA), torch.zeros_like(dA)
    g_D = torch.zeros(d, dtype=torch.float64)
    g = torch.zeros(batch, d, dtype=torch.float64)
    for t in range(seqlen - 1, -1, -1):
        g_C[:, t] = gy[:, t] * states[:, t + 1]
        g = g + gy[:, t] * C[:, t]
        g_D = g_D + (gy[:, t] * x[:, t]).sum(0)
        g_dA[:, t] = g * states[:, t]
        g_dBx[:, t] = g
        g = g * dA[:, t]
    return g_dA, g_dBx, g_C, g_D, gy * Dd
