"""CPU stand-in for the gfx950 launchers, built on the oracle (tests only).

``install(monkeypatch)`` replaces the tensor-level launchers in
``kernels.hip._lib`` with functions that compute the same outputs on the CPU
from ``oracle.ops`` and write them into the caller's output tensors, and
relaxes the GPU-device check. This lets the host logic (shape handling,
autograd wiring, the module registry) run in the CPU test tier. The product
never imports this module.
"""

import math

import torch
import torch.nn.functional as F

from oracle import ops


def _rmsnorm(x, w, y, eps):
    y.copy_(ops.rmsnorm_f32_ref(x, w, eps))


def _fused(x, r, w, nr, y, eps):
    hidden, out = ops.fused_residual_add_rmsnorm_ref(x, r, w, eps)
    if nr is not None:
        nr.copy_(hidden)
    y.copy_(out)


def _rmsnorm_bwd(x, w, g, gx, gw, ws, eps):
    a, b = ops.rmsnorm_bwd_ref(x, w, g, eps)
    gx.copy_(a.to(gx.dtype))
    if gw is not None:
        gw.copy_(b.float())


def _fused_bwd(h, w, gh, gn, gx, gw, ws, eps):
    a, b = ops.fused_residual_rmsnorm_bwd_ref(h, w, gh, gn, eps)
    gx.copy_(a.to(gx.dtype))
    if gw is not None:
        gw.copy_(b.float())


def _softmax(x, y):
    y.copy_(ops.softmax_ref(x))


def _bad_targets(targets, vocab, ignore_index):
    t = targets.long()
    return (t != ignore_index) & ((t < 0) | (t >= vocab))


def _ce_fwd(logits, targets, losses, lse, row_max, row_sum, grad, softcap, ignore_index, ls, scale,
            scale_dev=None, z_loss_weight=0.0):
    bad = _bad_targets(targets, logits.shape[1], ignore_index)
    t = torch.where(bad, torch.full_like(targets, ignore_index), targets)
    l, s, m, sm = ops.ce_rows_ref(logits, t, softcap, ignore_index, ls)
    l = torch.where(bad, torch.full_like(l, math.nan), l)
    losses.copy_(l)
    lse.copy_(s)
    if row_max is not None:
        row_max.copy_(m)
    if row_sum is not None:
        row_sum.copy_(sm)
    if grad is not None:
        sc = scale * (float(scale_dev.reshape(-1)[0]) if scale_dev is not None else 1.0)
        g = ops.ce_grad_ref(logits, t, softcap, ignore_index, ls, sc, z_loss_weight)
        g[bad] = math.nan
        grad.copy_(g)


def _ce_bwd_tiny(logits, targets, row_max, row_sum, grad, softcap, ignore_index, ls, scale,
                 z_loss_weight=0.0, scale_dev=None):
    sc = scale * (float(scale_dev.reshape(-1)[0]) if scale_dev is not None else 1.0)
    x = logits.float()
    if softcap > 0:
        x = softcap * torch.tanh(x / softcap)
    V = x.shape[1]
    p = torch.exp(x - row_max.float()[:, None]) / row_sum.float()[:, None]
    if z_loss_weight > 0:
        lse = row_max.float() + torch.log(row_sum.float())
        p = p * (1 + 2 * z_loss_weight * lse[:, None])
    t = targets.long()
    ignored = t == ignore_index
    tc = torch.where(ignored, torch.zeros_like(t), t)
    g = p - F.one_hot(tc, V).float() * (1 - ls)
    if ls > 0:
        g = g - ls / V
    if softcap > 0:
        th = x / softcap
        g = g * (1 - th * th)
    g = torch.where(ignored[:, None], torch.zeros_like(g), g * sc)
    grad.copy_(g)


def _ce_count_valid(targets, ignore_index):
    n = max(1, int((targets != ignore_index).sum()))
    return torch.tensor([float(n), 1.0 / n], dtype=torch.float32)


def _ce_mean(losses, lse, targets, ignore_index, z_loss_weight=0.0, n_valid=None):
    if n_valid is not None:
        n_valid.copy_((targets != ignore_index).sum().reshape(1))
    return ops.ce_mean_ref(losses, targets, ignore_index, lse, z_loss_weight)


def _lmhead(hidden, weight, targets, loss, lse, losses, n_valid, ws, ignore_index, softcap=0.0,
            label_smoothing=0.0):
    lo, ls_, per = ops.lmhead_ce_ref(hidden, weight, targets, ignore_index, softcap=softcap,
                                     label_smoothing=label_smoothing)
    bad = _bad_targets(targets, weight.shape[0], ignore_index)
    per = torch.where(bad, torch.full_like(per, math.nan), per)
    lo = ops.ce_mean_ref(per, targets, ignore_index)
    loss.copy_(lo)
    lse.copy_(ls_)
    if losses is not None:
        losses.copy_(per)
    if n_valid is not None:
        n_valid.copy_((targets != ignore_index).sum().reshape(1))


def _lmhead_bwd(hidden, weight, targets, lse, grad_loss, denom, grad_logits, ignore_index,
                softcap=0.0, label_smoothing=0.0):
    z = hidden.double() @ weight.double().t()
    dcap = torch.ones_like(z)
    if softcap > 0:
        th = torch.tanh(z / softcap)
        z, dcap = softcap * th, 1 - th * th
    p = torch.exp(z - lse.double()[:, None])
    t = targets.long()
    V = weight.shape[0]
    ok = (t >= 0) & (t < V)
    oh = F.one_hot(torch.where(ok, t, torch.zeros_like(t)), V).double() * ok[:, None]
    p = p - (1 - label_smoothing) * oh - label_smoothing / V
    g = p * dcap * (float(grad_loss.reshape(-1)[0]) / float(denom.reshape(-1)[0]))
    g = torch.where((t == ignore_index)[:, None], torch.zeros_like(g), g)
    g = torch.where((~ok & (t != ignore_index))[:, None], torch.full_like(g, math.nan), g)
    grad_logits[:, :V].copy_(g)


def _lmhead_bwd_range(hidden, weight, targets, lse, grad_loss, denom, grad_logits, v_begin,
                      ignore_index, softcap=0.0, label_smoothing=0.0):
    full = torch.empty((hidden.shape[0], weight.shape[0]), dtype=grad_logits.dtype)
    _lmhead_bwd(hidden, weight, targets, lse, grad_loss, denom, full, ignore_index, softcap,
                label_smoothing)
    grad_logits.copy_(full[:, v_begin:v_begin + grad_logits.shape[1]])


def _grad_gemm_out(out, val, out_mode):
    if out_mode == 2:
        out.add_(val.float())
    else:
        out.copy_(val.to(out.dtype))


def _grad_hidden(grad_logits, weight, out, out_mode, workspace):
    _grad_gemm_out(out, grad_logits.double() @ weight.double(), out_mode)


def _grad_weight(grad_logits, hidden, out, out_mode, workspace):
    _grad_gemm_out(out, grad_logits.double().t() @ hidden.double(), out_mode)


def _scan(u, delta, A, B, C, D, z, delta_bias, out, last_state, delta_softplus, out_prez=None,
          chunk_states=None, checkpoints=None):
    if A.is_complex():
        o, last = ops.selective_scan_complex_ref(u, delta, A, B, C, D, z, delta_bias, delta_softplus,
                                                 return_last_state=True)
        out.copy_(o)
        if last_state is not None:
            last_state.copy_(last)
        if out_prez is not None:
            out_prez.copy_(ops.selective_scan_complex_ref(u, delta, A, B, C, D, None, delta_bias,
                                                          delta_softplus))
        if chunk_states is not None:
            chunk_states.copy_(ops.selective_scan_complex_chunk_states_ref(u, delta, A, B, delta_bias,
                                                                           delta_softplus))
        if checkpoints is not None:
            checkpoints.zero_()
        return
    o, last = ops.selective_scan_ref(u, delta, A, B, C, D, z, delta_bias, delta_softplus,
                                     return_last_state=True)
    out.copy_(o)
    if last_state is not None:
        last_state.copy_(last)
    if out_prez is not None:
        out_prez.copy_(ops.selective_scan_ref(u, delta, A, B, C, D, None, delta_bias, delta_softplus))
    if chunk_states is not None:
        chunk_states.copy_(ops.selective_scan_chunk_states_ref(u, delta, A, B, delta_bias, delta_softplus))
    if checkpoints is not None:  # the fake backward recomputes; mark the buffer as written
        checkpoints.zero_()


def _scan_bwd(u, delta, A, B, C, D, z, delta_bias, dout, du, ddelta, dA, dB, dC, dD, dz, dbias,
              delta_softplus, checkpoints=None, out_prez=None):
    bwd = ops.selective_scan_complex_bwd_ref if A.is_complex() else ops.selective_scan_bwd_ref
    outs = bwd(u, delta, A, B, C, dout, D, z, delta_bias, delta_softplus)
    for dst, src in zip((du, ddelta, dA, dB, dC, dD, dz, dbias), outs):
        if dst is not None:
            dst.copy_(src.to(dst.dtype))


def _diag(dA, dBx, C, D, x, y):
    y.copy_(ops.diag_scan_ref(dA, dBx, C, D, x))


def _diag_bwd(dA, dBx, C, D, x, gy, g_dA, g_dBx, g_C, g_D, g_x):
    outs = ops.diag_scan_bwd_ref(dA, dBx, C, D, x, gy)
    for dst, src in zip((g_dA, g_dBx, g_C, g_D, g_x), outs):
        dst.copy_(src.float())


def install(monkeypatch):
    from kernels.hip import _lib
    monkeypatch.setattr(_lib, "require_device", lambda *tensors: None)
    monkeypatch.setattr(_lib, "rmsnorm", _rmsnorm)
    monkeypatch.setattr(_lib, "fused_add_rmsnorm", _fused)
    monkeypatch.setattr(_lib, "rmsnorm_bwd", _rmsnorm_bwd)
    monkeypatch.setattr(_lib, "fused_add_rmsnorm_bwd", _fused_bwd)
    monkeypatch.setattr(_lib, "rmsnorm_bwd_workspace_bytes", lambda rows, cols: 256)
    monkeypatch.setattr(_lib, "softmax", _softmax)
    monkeypatch.setattr(_lib, "ce_fwd", _ce_fwd)
    monkeypatch.setattr(_lib, "ce_bwd_tiny", _ce_bwd_tiny)
    monkeypatch.setattr(_lib, "ce_count_valid", _ce_count_valid)
    monkeypatch.setattr(_lib, "ce_mean", _ce_mean)
    monkeypatch.setattr(_lib, "lmhead_ce", _lmhead)
    monkeypatch.setattr(_lib, "lmhead_ce_workspace_bytes", lambda n, v: 256)
    monkeypatch.setattr(_lib, "lmhead_ce_bwd", _lmhead_bwd)
    monkeypatch.setattr(_lib, "lmhead_ce_bwd_range", _lmhead_bwd_range)
    monkeypatch.setattr(_lib, "lmhead_grad_workspace_bytes", lambda n, v, d: 256)
    monkeypatch.setattr(_lib, "lmhead_grad_hidden", _grad_hidden)
    monkeypatch.setattr(_lib, "lmhead_grad_weight", _grad_weight)
    monkeypatch.setattr(_lib, "selective_scan", _scan)
    monkeypatch.setattr(_lib, "selective_scan_bwd", _scan_bwd)
    monkeypatch.setattr(_lib, "diag_scan", _diag)
    monkeypatch.setattr(_lib, "diag_scan_bwd", _diag_bwd)
