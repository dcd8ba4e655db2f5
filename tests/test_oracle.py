"""Pins the CPU oracle (CPU tier).

Each oracle function is checked against something it does not itself
compute: closed forms, invariants, torch's own independent implementations
(F.cross_entropy and its autograd, torch.logsumexp), float64 brute force on
tiny inputs, an independent bf16 round-to-nearest-even, and the reference's
known-answer test (tests/golden/griffin_kat.json). The checks are chosen so
that a dropped term, a wrong sign or index, or a transposed operand fails.
"""

import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import c_oracle, ops

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _bf16_rne(x32: torch.Tensor) -> torch.Tensor:
    """fp32 -> bf16 round-to-nearest-even by integer arithmetic (finite inputs)."""
    b = x32.contiguous().numpy().view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return torch.from_numpy(r.view(np.float32).copy()).bfloat16()


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------

def test_rmsnorm_known_answer():
    x = torch.tensor([[3.0, 4.0]])
    r = math.sqrt(12.5)
    y = ops.rmsnorm_ref(x, torch.tensor([1.0, 1.0]), eps=0.0)
    assert torch.allclose(y, torch.tensor([[3 / r, 4 / r]]), rtol=1e-6)
    y = ops.rmsnorm_ref(x, torch.tensor([2.0, 0.5]), eps=0.0)
    assert torch.allclose(y, torch.tensor([[6 / r, 2 / r]]), rtol=1e-6)
    # eps enters under the square root
    y = ops.rmsnorm_ref(x, torch.tensor([1.0, 1.0]), eps=0.5)
    assert torch.allclose(y, torch.tensor([[3 / math.sqrt(13.0), 4 / math.sqrt(13.0)]]), rtol=1e-6)


def test_rmsnorm_invariants():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(16, 96, generator=g)
    w = torch.ones(96)
    y = ops.rmsnorm_ref(x, w, eps=0.0)
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(16), rtol=1e-5)   # unit RMS per row
    assert torch.allclose(ops.rmsnorm_ref(7.3 * x, w, 0.0), y, rtol=1e-5, atol=1e-6)  # scale invariance
    assert torch.equal(ops.rmsnorm_ref(torch.zeros(2, 8), torch.ones(8)), torch.zeros(2, 8))
    assert torch.equal(ops.rmsnorm_f32_ref(x, w, 1e-6), ops.rmsnorm_ref(x, w, 1e-6))


def test_rmsnorm_brute_force_f64():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(3, 5, generator=g)
    w = torch.randn(5, generator=g)
    y = ops.rmsnorm_f32_ref(x, w, 1e-6)
    for i in range(3):
        ms = sum(float(v) ** 2 for v in x[i]) / 5
        for j in range(5):
            assert abs(float(y[i, j]) - float(x[i, j]) / math.sqrt(ms + 1e-6) * float(w[j])) < 1e-5


@pytest.mark.parametrize("eps", [1e-6, 1e-5, 0.3])
def test_rmsnorm_bwd_matches_autograd(eps):
    """The oracle's backward equals torch autograd of the float64 forward
    (reference.py:25-29); the reference's own PyTorch fallback formula
    (_torch_ops.py:95, which drops one factor of 1/rms in the projection
    term) does not."""
    g = torch.Generator().manual_seed(11)
    x = (3 * torch.randn(6, 40, generator=g)).double().requires_grad_(True)
    w = (1 + 0.1 * torch.randn(40, generator=g)).double().requires_grad_(True)
    dy = torch.randn(6, 40, generator=g).double()
    ops.rmsnorm_ref(x, w, eps).backward(dy)
    gx, gw = ops.rmsnorm_bwd_ref(x.detach(), w.detach(), dy, eps)
    assert torch.allclose(gx, x.grad, rtol=1e-12, atol=1e-12)
    assert torch.allclose(gw, w.grad, rtol=1e-12, atol=1e-12)
    # the fallback formula of the reference's _torch_ops.py:95
    xd = x.detach()
    r = (xd.pow(2).mean(-1, keepdim=True) + eps).rsqrt()
    n = xd * r
    gn = dy * w.detach()
    wrong = gn * r - n * (gn * n).sum(-1, keepdim=True) / 40
    assert not torch.allclose(wrong, x.grad, rtol=1e-3, atol=1e-3)


def test_rmsnorm_bwd_closed_forms():
    g = torch.Generator().manual_seed(12)
    x = torch.randn(5, 64, generator=g).double()
    w = torch.randn(64, generator=g).double()
    dy = torch.randn(5, 64, generator=g).double()
    gx, gw = ops.rmsnorm_bwd_ref(x, w, dy, 0.0)
    # zero upstream gradient -> zero gradients
    z = ops.rmsnorm_bwd_ref(x, w, torch.zeros_like(dy), 0.0)
    assert torch.equal(z[0], torch.zeros_like(x)) and torch.equal(z[1], torch.zeros(64, dtype=torch.float64))
    # with eps = 0 the output is scale invariant, so the gradient is orthogonal
    # to x row by row and scales as 1/c under x -> c x
    assert torch.allclose((gx * x).sum(-1), torch.zeros(5, dtype=torch.float64), atol=1e-10)
    gx2, gw2 = ops.rmsnorm_bwd_ref(4.0 * x, w, dy, 0.0)
    assert torch.allclose(gx2, gx / 4.0, rtol=1e-12, atol=1e-14)
    assert torch.allclose(gw2, gw, rtol=1e-12, atol=1e-14)
    # grad_weight is the column sum of dy * (x / rms), by brute force
    for j in (0, 17, 63):
        s = 0.0
        for i in range(5):
            rms = math.sqrt(sum(float(v) ** 2 for v in x[i]) / 64)
            s += float(dy[i, j]) * float(x[i, j]) / rms
        assert abs(float(gw[j]) - s) < 1e-10


def test_fused_rmsnorm_bwd_matches_autograd():
    """grad_x = grad_residual = grad_hidden + norm backward, against autograd of
    the dual-output forward (hidden, rmsnorm(hidden)) in float64."""
    g = torch.Generator().manual_seed(13)
    x = torch.randn(4, 48, generator=g).double().requires_grad_(True)
    r = torch.randn(4, 48, generator=g).double().requires_grad_(True)
    w = (1 + 0.1 * torch.randn(48, generator=g)).double().requires_grad_(True)
    gh = torch.randn(4, 48, generator=g).double()
    gn = torch.randn(4, 48, generator=g).double()
    hidden = x + r
    y = ops.rmsnorm_ref(hidden, w, 1e-5)
    torch.autograd.backward([hidden, y], [gh, gn])
    gx, gw = ops.fused_residual_rmsnorm_bwd_ref(hidden.detach(), w.detach(), gh, gn, 1e-5)
    assert torch.allclose(gx, x.grad, rtol=1e-12, atol=1e-12)
    assert torch.allclose(gx, r.grad, rtol=1e-12, atol=1e-12)
    assert torch.allclose(gw, w.grad, rtol=1e-12, atol=1e-12)
    gx0, _ = ops.fused_residual_rmsnorm_bwd_ref(hidden.detach(), w.detach(), None, gn, 1e-5)
    assert torch.allclose(gx0 + gh, gx, rtol=1e-12, atol=1e-12)


def test_fused_hidden_is_rne_of_exact_sum():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, 256, generator=g).bfloat16()
    r = torch.randn(64, 256, generator=g).bfloat16()
    w = (1 + 0.02 * torch.randn(256, generator=g)).bfloat16()
    hidden, y = ops.fused_residual_add_rmsnorm_ref(x, r, w, 1e-5)
    assert torch.equal(hidden, _bf16_rne(x.float() + r.float()))
    # a tie rounds to even: 1 + 2^-8 lies halfway between bf16 1.0 and 1.0078125
    h, _ = ops.fused_residual_add_rmsnorm_ref(torch.tensor([[1.0]]).bfloat16(),
                                              torch.tensor([[2.0 ** -8]]).bfloat16(),
                                              torch.ones(1).bfloat16())
    assert float(h) == 1.0
    # the norm is taken of the rounded sum, not of x alone
    assert torch.equal(y, ops.rmsnorm_f32_ref(hidden, w, 1e-5))
    assert not torch.equal(y, ops.rmsnorm_f32_ref(x, w, 1e-5))


# ---------------------------------------------------------------------------
# Softmax
# ---------------------------------------------------------------------------

def test_softmax_known_answer_and_mask():
    y = ops.softmax_ref(torch.tensor([[0.0, math.log(2), math.log(3)]]))
    assert torch.allclose(y, torch.tensor([[1 / 6, 1 / 3, 1 / 2]]), rtol=1e-6)
    g = torch.Generator().manual_seed(4)
    S = 16
    x = (3 * torch.randn(2, 3, S, S, generator=g)).half()
    x = x.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    y = ops.softmax_ref(x)
    assert y.dtype == torch.float16
    nz = (y != 0).sum(-1)
    assert torch.equal(nz, torch.arange(1, S + 1).expand(2, 3, S))     # row i: i+1 non-zeros
    assert bool((y[..., 0, 0] == 1.0).all())                             # row 0 is exactly 1
    eq = torch.zeros(S, S).masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    ye = ops.softmax_ref(eq)
    for i in range(S):
        assert torch.allclose(ye[i, : i + 1], torch.full((i + 1,), 1.0 / (i + 1)))


def test_softmax_invariants():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(32, 100, generator=g)
    y = ops.softmax_ref(x)
    assert torch.allclose(y.sum(-1), torch.ones(32), atol=1e-6)
    assert torch.allclose(ops.softmax_ref(x + 11.0), y, atol=1e-6)


# ---------------------------------------------------------------------------
# Cross-entropy
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("ls", [0.0, 0.1])
def test_ce_rows_match_torch_cross_entropy(ls):
    g = torch.Generator().manual_seed(6)
    logits = 3 * torch.randn(24, 37, generator=g)
    t = torch.randint(0, 37, (24,), generator=g)
    t[[1, 5, 7]] = -100
    losses, lse, _, _ = ops.ce_rows_ref(logits, t, 0.0, -100, ls)
    ref = F.cross_entropy(logits.double(), t, ignore_index=-100, label_smoothing=ls, reduction="none")
    assert torch.allclose(losses.double(), ref, rtol=1e-5, atol=1e-5)
    assert torch.allclose(lse.double(), torch.logsumexp(logits.double(), -1), rtol=1e-6)
    mean = ops.ce_mean_ref(losses, t)
    assert torch.allclose(mean.double(), F.cross_entropy(logits.double(), t, label_smoothing=ls), rtol=1e-5)


@pytest.mark.parametrize("softcap,ls", [(0.0, 0.0), (0.0, 0.2), (5.0, 0.0), (5.0, 0.1)])
def test_ce_grad_matches_autograd(softcap, ls):
    g = torch.Generator().manual_seed(7)
    logits = (4 * torch.randn(10, 13, generator=g)).double().requires_grad_()
    t = torch.randint(0, 13, (10,), generator=g)
    t[3] = -100
    x = softcap * torch.tanh(logits / softcap) if softcap > 0 else logits
    loss = F.cross_entropy(x, t, ignore_index=-100, label_smoothing=ls)
    loss.backward()
    n_valid = int((t != -100).sum())
    grad = ops.ce_grad_ref(logits.detach().float(), t, softcap, -100, ls, 1.0 / n_valid)
    assert torch.allclose(grad.double(), logits.grad, atol=2e-6, rtol=1e-4)
    losses, _, _, _ = ops.ce_rows_ref(logits.detach().float(), t, softcap, -100, ls)
    assert torch.allclose(ops.ce_mean_ref(losses, t).double(), loss.detach(), rtol=1e-5)


@pytest.mark.parametrize("softcap,ls", [(0.0, 0.0), (6.0, 0.0), (6.0, 0.15)])
def test_ce_zloss_grad_and_mean_match_autograd(softcap, ls):
    # loss = mean over counted rows of (CE + w * lse^2): float64 autograd pins
    # both the z-loss term of ce_mean_ref and the 2 w lse p term of ce_grad_ref,
    # including the softcap's chain rule
    w = 0.03
    g = torch.Generator().manual_seed(17)
    logits = (4 * torch.randn(9, 21, generator=g)).double().requires_grad_()
    t = torch.randint(0, 21, (9,), generator=g)
    t[[2, 6]] = -100
    x = softcap * torch.tanh(logits / softcap) if softcap > 0 else logits
    valid = (t != -100).double()
    ce = F.cross_entropy(x, t, ignore_index=-100, label_smoothing=ls)
    loss = ce + w * (torch.logsumexp(x, -1) ** 2 * valid).sum() / valid.sum()
    loss.backward()
    grad = ops.ce_grad_ref(logits.detach().float(), t, softcap, -100, ls, 1.0 / 7, w)
    assert torch.allclose(grad.double(), logits.grad, atol=3e-6, rtol=1e-4)
    losses, lse, _, _ = ops.ce_rows_ref(logits.detach().float(), t, softcap, -100, ls)
    mean = ops.ce_mean_ref(losses, t, -100, lse, w)
    assert torch.allclose(mean.double(), loss.detach(), rtol=1e-5)
    # the z-loss term really enters: without it the gradient differs
    plain = ops.ce_grad_ref(logits.detach().float(), t, softcap, -100, ls, 1.0 / 7)
    assert not torch.allclose(plain.double(), logits.grad, atol=1e-4)


def test_ce_closed_forms():
    V = 50
    losses, lse, _, _ = ops.ce_rows_ref(torch.zeros(4, V), torch.tensor([0, 3, 49, 7]))
    assert torch.allclose(lse, torch.full((4,), math.log(V)))
    assert torch.allclose(losses, torch.full((4,), math.log(V)))
    t = torch.full((4,), -100)
    losses, _, _, _ = ops.ce_rows_ref(torch.randn(4, V), t)
    assert float(ops.ce_mean_ref(losses, t)) == 0.0
    x = torch.randn(4, V)
    tt = torch.tensor([1, 2, 3, 4])
    l0, s0, _, _ = ops.ce_rows_ref(x, tt)
    l1, s1, _, _ = ops.ce_rows_ref(x + 9.0, tt)
    assert torch.allclose(s1, s0 + 9.0, atol=1e-5) and torch.allclose(l1, l0, atol=1e-5)


def test_lmhead_ce_ref_matches_materialised():
    g = torch.Generator().manual_seed(8)
    h = torch.randn(40, 64, generator=g)
    W = 0.1 * torch.randn(1000, 64, generator=g)
    t = torch.randint(0, 1000, (40,), generator=g)
    t[[0, 9]] = -100
    loss, lse, losses = ops.lmhead_ce_ref(h, W, t, vocab_chunk=4096)
    logits = h.double() @ W.double().t()
    assert torch.allclose(lse.double(), torch.logsumexp(logits, -1), rtol=1e-6)
    assert torch.allclose(loss.double(), F.cross_entropy(logits, t), rtol=1e-5)
    for chunk in (7, 256, 333):
        l2, s2, _ = ops.lmhead_ce_ref(h, W, t, vocab_chunk=chunk)
        assert torch.allclose(s2, lse, rtol=1e-6) and torch.allclose(l2, loss, rtol=1e-6)


@pytest.mark.parametrize("softcap,ls", [(0.0, 0.0), (5.0, 0.0), (0.0, 0.2), (5.0, 0.2)])
def test_lmhead_ce_ref_float64_matches_torch(softcap, ls):
    """The float64 mode (used for the full-size C4 checks) against
    F.cross_entropy / logsumexp of the float64 logits, to float64 rounding,
    for every vocab chunking; a wrong merge of the chunk partials, a dropped
    smoothing or softcap term, or a float32 step inside would miss 1e-12."""
    g = torch.Generator().manual_seed(29)
    h = torch.randn(64, 48, generator=g)
    W = 0.5 * torch.randn(700, 48, generator=g)
    t = torch.randint(0, 700, (64,), generator=g)
    t[[1, 40]] = -100
    z = h.double() @ W.double().t()
    if softcap > 0:
        z = softcap * torch.tanh(z / softcap)
    ref = F.cross_entropy(z, t, label_smoothing=ls)
    ref_per = F.cross_entropy(z, t, label_smoothing=ls, reduction="none")
    for chunk in (64, 333, 4096):
        loss, lse, per = ops.lmhead_ce_ref(h, W, t, vocab_chunk=chunk, softcap=softcap,
                                           label_smoothing=ls, dtype=torch.float64)
        assert lse.dtype == per.dtype == loss.dtype == torch.float64
        assert torch.allclose(lse, torch.logsumexp(z, -1), rtol=1e-12, atol=0)
        assert torch.allclose(per, ref_per, rtol=1e-12, atol=1e-12)
        assert abs(float(loss) - float(ref)) <= 1e-12 * abs(float(ref))


# ---------------------------------------------------------------------------
# Scans
# ---------------------------------------------------------------------------

def _kat():
    with open(os.path.join(GOLDEN, "griffin_kat.json")) as f:
        return json.load(f)


def test_diag_scan_known_answer():
    k = _kat()
    dA = torch.tensor(k["decay"]).view(1, 4, 1)
    dBx = torch.tensor(k["value"]).view(1, 4, 1)
    y = ops.diag_scan_ref(dA, dBx, torch.ones(1, 4, 1), torch.zeros(1), torch.zeros(1, 4, 1))
    assert torch.allclose(y.view(-1), torch.tensor(k["expected"]), rtol=1e-6)
    x = torch.randn(1, 4, 1)
    y = ops.diag_scan_ref(dA, dBx, torch.zeros(1, 4, 1), torch.full((1,), 2.5), x)
    assert torch.allclose(y, 2.5 * x)


def test_selective_scan_known_answer():
    """KAT mapped to N=1: A=-1, delta_t = -ln(a_t), B=C=1, D=None, u_t = b_t / delta_t."""
    k = _kat()
    a = torch.tensor(k["decay"], dtype=torch.float64)
    delta = (-torch.log(a)).float().view(1, 1, 4)
    u = (torch.tensor(k["value"], dtype=torch.float64) / -torch.log(a)).float().view(1, 1, 4)
    A = torch.tensor([[-1.0]])
    B = torch.ones(1, 1, 4)
    y = ops.selective_scan_ref(u, delta, A, B, B.clone())
    assert torch.allclose(y.view(-1), torch.tensor(k["expected"]), rtol=1e-5)
    yc, _ = c_oracle.selective_scan(u, delta, A, B, B.clone())
    assert torch.allclose(yc.view(-1), torch.tensor(k["expected"]), rtol=1e-5)


def _scan_inputs(b=2, d=4, l=32, n=8, g=1, seed=9):
    gen = torch.Generator().manual_seed(seed)
    u = torch.randn(b, d, l, generator=gen)
    delta = 0.5 * torch.rand(b, d, l, generator=gen)
    A = -0.5 * torch.rand(d, n, generator=gen) - 0.1
    B = torch.randn(b, g, n, l, generator=gen)
    C = torch.randn(b, g, n, l, generator=gen)
    D = torch.randn(d, generator=gen)
    z = torch.randn(b, d, l, generator=gen)
    bias = 0.5 * torch.rand(d, generator=gen)
    return u, delta, A, B, C, D, z, bias


def test_selective_scan_closed_forms():
    u, delta, A, B, C, D, z, bias = _scan_inputs()
    # delta = 0: no state, out = D * u * silu(z)
    out = ops.selective_scan_ref(u, torch.zeros_like(delta), A, B, C, D, z)
    assert torch.allclose(out, D[:, None] * u * F.silu(z), atol=1e-6)
    # A = 0: the state is a running sum of delta*u*B
    out = ops.selective_scan_ref(u, delta, torch.zeros_like(A), B, C)
    h = torch.cumsum((delta * u)[:, :, None, :] * B, dim=-1)          # [b, d, n, l] (g=1 broadcasts)
    assert torch.allclose(out, (h * C).sum(2), rtol=1e-4, atol=1e-5)
    # L = 1
    out = ops.selective_scan_ref(u[..., :1], delta[..., :1], A, B[..., :1], C[..., :1], D)
    y1 = (delta[..., :1] * u[..., :1])[:, :, None, :] * B[..., :1] * C[..., :1]
    assert torch.allclose(out, y1.sum(2) + D[:, None] * u[..., :1], atol=1e-6)


def test_selective_scan_invariants():
    u, delta, A, B, C, D, z, bias = _scan_inputs(l=40)
    u2 = torch.randn_like(u)
    lin = ops.selective_scan_ref(2 * u + 3 * u2, delta, A, B, C, D)
    sep = 2 * ops.selective_scan_ref(u, delta, A, B, C, D) + 3 * ops.selective_scan_ref(u2, delta, A, B, C, D)
    assert torch.allclose(lin, sep, rtol=1e-4, atol=1e-4)
    # split equivalence: scan(L) == scan(L/2) then continue from last_state
    full, last = ops.selective_scan_ref(u, delta, A, B, C, D, z, bias, True, return_last_state=True)
    h = 20
    a1, s1 = ops.selective_scan_ref(u[..., :h], delta[..., :h], A, B[..., :h], C[..., :h], D,
                                    z[..., :h], bias, True, return_last_state=True)
    a2, s2 = ops.selective_scan_ref(u[..., h:], delta[..., h:], A, B[..., h:], C[..., h:], D,
                                    z[..., h:], bias, True, return_last_state=True, initial_state=s1)
    assert torch.allclose(torch.cat([a1, a2], -1), full, rtol=1e-5, atol=1e-5)
    assert torch.allclose(s2, last, rtol=1e-5, atol=1e-6)
    # softplus / bias are applied to delta before everything else
    pre = ops.selective_scan_ref(u, F.softplus(delta + bias[:, None]), A, B, C, D, z)
    assert torch.allclose(pre, ops.selective_scan_ref(u, delta, A, B, C, D, z, bias, True), atol=1e-6)


def test_selective_scan_groups():
    u, delta, A, B, C, D, z, bias = _scan_inputs(d=8, g=2)
    out = ops.selective_scan_ref(u, delta, A, B, C, D, z)
    lo = ops.selective_scan_ref(u[:, :4], delta[:, :4], A[:4], B[:, 0], C[:, 0], D[:4], z[:, :4])
    hi = ops.selective_scan_ref(u[:, 4:], delta[:, 4:], A[4:], B[:, 1], C[:, 1], D[4:], z[:, 4:])
    assert torch.allclose(out, torch.cat([lo, hi], 1), atol=1e-6)


def test_c_oracle_matches_torch_oracle():
    for g in (1, 2):
        u, delta, A, B, C, D, z, bias = _scan_inputs(d=8, l=70, g=g, seed=10 + g)
        ref, last = ops.selective_scan_ref(u, delta, A, B, C, D, z, bias, True, return_last_state=True)
        out, lc = c_oracle.selective_scan(u, delta, A, B, C, D, z, bias, True)
        assert torch.allclose(out, ref, rtol=1e-5, atol=1e-5)
        assert torch.allclose(lc, last, rtol=1e-5, atol=1e-6)


def _scan_brute(u, delta, A, Bfn, Cfn, D=None, z=None, bias=None, softplus=False):
    """Scalar float64 loops over (b, d, l, n): h = exp(delta' A) h + delta' u B;
    y = sum_n h C + D u; out = y silu(z). Bfn / Cfn(b, d, n, l) give the B / C
    entry that channel d sees at step l (any layout)."""
    bsz, dim, L = u.shape
    N = A.shape[1]
    out = torch.zeros(bsz, dim, L, dtype=torch.float64)
    last = torch.zeros(bsz, dim, N, dtype=torch.float64)
    for b in range(bsz):
        for d in range(dim):
            h = [0.0] * N
            for l in range(L):
                x = float(delta[b, d, l]) + (float(bias[d]) if bias is not None else 0.0)
                if softplus:
                    x = x if x > 20 else math.log1p(math.exp(x))
                y = 0.0
                for n in range(N):
                    h[n] = math.exp(x * float(A[d, n])) * h[n] + x * float(u[b, d, l]) * Bfn(b, d, n, l)
                    y += h[n] * Cfn(b, d, n, l)
                if D is not None:
                    y += float(D[d]) * float(u[b, d, l])
                if z is not None:
                    zz = float(z[b, d, l])
                    y *= zz / (1 + math.exp(-zz))
                out[b, d, l] = y
            last[b, d] = torch.tensor(h, dtype=torch.float64)
    return out, last


@pytest.mark.parametrize("layout", ["const_B", "const_C", "const_BC", "wide_var"])
def test_selective_scan_input_independent_bc_and_wide_state_brute_force(layout):
    """Input-independent B / C ([dim, n], selective_scan_interface.py:151-152,
    :168-169) and dstate 20 (past 16) against scalar float64 loops."""
    n = 20 if layout == "wide_var" else 6
    u, delta, A, B, C, D, z, bias = _scan_inputs(b=2, d=3, l=11, n=n, seed=61)
    gen = torch.Generator().manual_seed(62)
    B2, C2 = torch.randn(3, n, generator=gen), torch.randn(3, n, generator=gen)
    Bv = lambda b, d, k, l: float(B[b, 0, k, l])
    Cv = lambda b, d, k, l: float(C[b, 0, k, l])
    Bk = lambda b, d, k, l: float(B2[d, k])
    Ck = lambda b, d, k, l: float(C2[d, k])
    Bt, Bf = (B2, Bk) if layout in ("const_B", "const_BC") else (B[:, 0], Bv)
    Ct, Cf = (C2, Ck) if layout in ("const_C", "const_BC") else (C[:, 0], Cv)
    out, last = ops.selective_scan_ref(u, delta, A, Bt, Ct, D, z, bias, True, return_last_state=True)
    ref, rlast = _scan_brute(u, delta, A, Bf, Cf, D, z, bias, True)
    assert torch.allclose(out.double(), ref, rtol=1e-5, atol=1e-5)
    assert torch.allclose(last.double(), rlast, rtol=1e-5, atol=1e-5)
    c_out, c_last = c_oracle.selective_scan(u, delta, A, Bt, Ct, D, z, bias, True)
    assert torch.allclose(c_out.double(), ref, rtol=1e-5, atol=1e-5)
    assert torch.allclose(c_last.double(), rlast, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("const_b,const_c", [(True, False), (False, True), (True, True)])
def test_selective_scan_bwd_input_independent_bc_matches_autograd(const_b, const_c):
    """dB / dC of an input-independent B / C (summed over batch and steps) and
    every other gradient, against torch autograd of the float64 forward, with a
    grouped input-dependent partner (2 groups) and dstate 18."""
    u, delta, A, B, C, D, z, bias = _scan_inputs(d=4, l=23, n=18, g=2, seed=71)
    gen = torch.Generator().manual_seed(72)
    Bt = torch.randn(4, 18, generator=gen) if const_b else B
    Ct = torch.randn(4, 18, generator=gen) if const_c else C
    dout = torch.randn(u.shape, generator=gen)
    leaves = [t.double().requires_grad_() for t in (u, delta, A, Bt, Ct, D, z, bias)]
    out = ops.selective_scan_ref(*leaves[:5], D=leaves[5], z=leaves[6], delta_bias=leaves[7],
                                 delta_softplus=True, compute_dtype=torch.float64)
    out.backward(dout.double())
    ref = ops.selective_scan_bwd_ref(u, delta, A, Bt, Ct, dout, D, z, bias, True)
    for name, r, leaf in zip("du ddelta dA dB dC dD dz dbias".split(), ref, leaves):
        assert r.shape == leaf.grad.shape, name
        assert torch.allclose(r, leaf.grad, rtol=1e-10, atol=1e-12), name


def test_silu_dtype_choice_is_rounding_only():
    u, delta, A, B, C, D, z, bias = _scan_inputs()
    zb = z.bfloat16()
    a = ops.selective_scan_ref(u, delta, A, B, C, D, zb, silu_fp32=True)
    b = ops.selective_scan_ref(u, delta, A, B, C, D, zb, silu_fp32=False)
    assert torch.allclose(a, b, rtol=1e-2, atol=1e-2)


def test_diag_scan_bwd_matches_autograd():
    """The restated sequential backward (_torch_ops.py:346-386) equals torch
    autograd of the float64 forward recurrence."""
    g = torch.Generator().manual_seed(31)
    shp = (3, 17, 5)
    ins = [torch.rand(*shp, generator=g).double(), torch.randn(*shp, generator=g).double(),
           torch.randn(*shp, generator=g).double(), torch.randn(5, generator=g).double(),
           torch.randn(*shp, generator=g).double()]
    gy = torch.randn(*shp, generator=g).double()
    req = [t.clone().requires_grad_() for t in ins]
    dA, dBx, C, D, x = req
    s = torch.zeros(3, 5, dtype=torch.float64)
    ys = []
    for t in range(17):
        s = dA[:, t] * s + dBx[:, t]
        ys.append(C[:, t] * s + D * x[:, t])
    torch.stack(ys, 1).backward(gy)
    outs = ops.diag_scan_bwd_ref(*ins, gy)
    for got, t in zip(outs, req):
        assert torch.allclose(got, t.grad, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("softplus,gated,groups", [(False, False, 1), (True, True, 1), (True, True, 2),
                                                    (False, True, 2)])
def test_selective_scan_bwd_matches_autograd(softplus, gated, groups):
    """The restated reverse recurrence (selective_scan_bwd_kernel.cuh:189-300,
    :452-455) equals torch autograd of the float64 forward oracle, every
    gradient, with and without gate, skip, bias and softplus."""
    u, delta, A, B, C, D, z, bias = _scan_inputs(d=4, l=37, g=groups, seed=41 + groups)
    if softplus:
        delta = delta - 1.0  # around softplus' bend
    dout = torch.randn(u.shape, generator=torch.Generator().manual_seed(5))
    opt = (D, z, bias) if gated else (None, None, None)
    leaves = [t.double().requires_grad_() for t in (u, delta, A, B, C)]
    oleaves = [None if t is None else t.double().requires_grad_() for t in opt]
    out = ops.selective_scan_ref(*leaves, D=oleaves[0], z=oleaves[1], delta_bias=oleaves[2],
                                 delta_softplus=softplus, compute_dtype=torch.float64)
    assert out.dtype == torch.float64
    out.backward(dout.double())
    ref = ops.selective_scan_bwd_ref(u, delta, A, B, C, dout, *opt, delta_softplus=softplus)
    auto = [t.grad for t in leaves] + [None if t is None else t.grad for t in oleaves]
    for name, r, a in zip("du ddelta dA dB dC dD dz dbias".split(), ref, auto):
        if a is None:
            assert r is None, name
            continue
        assert r.shape == a.shape, name
        assert torch.allclose(r, a, rtol=1e-10, atol=1e-12), name


def test_selective_scan_bwd_softplus_threshold_and_closed_forms():
    """Special cases fixed by the mathematics: above softplus' threshold
    (20) ddelta = ddelta'; with A = 0 and one step, du = D dy + dy sum_n C B
    delta and dB = dy C delta u (dC = dy delta u B); with dout = 0 every
    gradient is zero; a 3-D B / C gives 3-D dB / dC."""
    u, delta, A, B, C, D, z, bias = _scan_inputs(l=9)
    dout = torch.randn(u.shape, generator=torch.Generator().manual_seed(6))
    big = delta + 25.0
    sp = ops.selective_scan_bwd_ref(u, big, A, B, C, dout, delta_softplus=True)
    nosp = ops.selective_scan_bwd_ref(u, big, A, B, C, dout, delta_softplus=False)
    assert torch.allclose(sp[1], nosp[1], rtol=1e-12, atol=1e-12)
    u1, d1, B1, C1 = u[..., :1], delta[..., :1], B[..., :1], C[..., :1]
    g1 = dout[..., :1]
    du, ddl, dA, dB, dC, dD, dz, db = ops.selective_scan_bwd_ref(u1, d1, torch.zeros_like(A), B1, C1, g1, D)
    cb = (C1 * B1).sum(2).double()                                     # [b, 1, 1] (g = 1)
    assert torch.allclose(du, D[:, None].double() * g1.double() + g1.double() * cb * d1.double())
    assert torch.allclose(ddl, g1.double() * u1.double() * cb)
    assert torch.allclose(dB[:, 0], (g1.double() * d1.double() * u1.double()).sum(1, keepdim=True)
                          * C1[:, 0].double())
    assert torch.allclose(dC[:, 0], (g1.double() * d1.double() * u1.double()).sum(1, keepdim=True)
                          * B1[:, 0].double())
    zero = ops.selective_scan_bwd_ref(u, delta, A, B, C, torch.zeros_like(dout), D, z, bias, True)
    assert all(float(t.abs().max()) == 0.0 for t in zero)
    out3 = ops.selective_scan_bwd_ref(u, delta, A, B[:, 0], C[:, 0], dout)
    assert out3[3].shape == B[:, 0].shape and out3[4].shape == C[:, 0].shape


def test_selective_scan_chunk_states_pinned():
    """Chunk states (selective_scan.cpp:307-313): the state entry of chunk k
    is the forward oracle's last_state over the prefix ending at chunk k; the
    decay entry is the last_state of a scan with u = 0 started from ones
    (h = prod a * h0). Chunk length 16 here, 2048 in the kernels."""
    u, delta, A, B, C, D, z, bias = _scan_inputs(l=40, g=2, seed=12)
    xs = ops.selective_scan_chunk_states_ref(u, delta, A, B, bias, True, chunk=16)
    assert xs.shape == (2, 4, 3, 8, 2)
    for k, end in enumerate((16, 32, 40)):
        _, last = ops.selective_scan_ref(u[..., :end], delta[..., :end], A, B[..., :end], C[..., :end],
                                         None, None, bias, True, return_last_state=True,
                                         compute_dtype=torch.float64)
        assert torch.allclose(xs[:, :, k, :, 1], last, rtol=1e-12, atol=1e-12)
        _, prod = ops.selective_scan_ref(torch.zeros_like(u[..., :end]), delta[..., :end], A,
                                         B[..., :end], C[..., :end], None, None, bias, True,
                                         return_last_state=True,
                                         initial_state=torch.ones(2, 4, 8, dtype=torch.float64),
                                         compute_dtype=torch.float64)
        assert torch.allclose(xs[:, :, k, :, 0], prod, rtol=1e-12, atol=1e-300)


def _complex_scan_inputs(b=2, d=4, l=24, n=6, g=1, seed=51, const_b=False, const_c=False):
    """Complex-A inputs in the reference's layouts: A complex [d, n] (S4D-like:
    negative real part, imaginary part pi * k), a variable B / C real
    [b, g, n, 2l] of (re, im) pairs, a constant one complex [d, n]."""
    gen = torch.Generator().manual_seed(seed)
    u = torch.randn(b, d, l, generator=gen)
    delta = 0.5 * torch.rand(b, d, l, generator=gen)
    Ar = -0.5 * torch.rand(d, n, generator=gen) - 0.1
    Ai = math.pi * torch.arange(n, dtype=torch.float32)[None].expand(d, n) * (0.5 + torch.rand(d, n, generator=gen))
    A = torch.complex(Ar, Ai)
    bc = lambda const: (torch.complex(torch.randn(d, n, generator=gen), torch.randn(d, n, generator=gen))
                        if const else torch.randn(b, g, n, 2 * l, generator=gen))
    B, C = bc(const_b), bc(const_c)
    D = torch.randn(d, generator=gen)
    z = torch.randn(b, d, l, generator=gen)
    bias = 0.5 * torch.rand(d, generator=gen)
    return u, delta, A, B, C, D, z, bias


def test_complex_scan_real_reduction():
    """With Im A = 0 and real B / C the complex scan is twice the real one
    (y = 2 Re sum h C, selective_scan_interface.py:173-174), D u added after
    the doubling."""
    u, delta, A, B, C, D, z, bias = _complex_scan_inputs(seed=52)
    Ar = A.real.contiguous()
    Bre, Cre = B[..., 0::2], C[..., 0::2]
    Bc = torch.stack([Bre, torch.zeros_like(Bre)], -1).reshape(B.shape)
    Cc = torch.stack([Cre, torch.zeros_like(Cre)], -1).reshape(C.shape)
    got = ops.selective_scan_complex_ref(u, delta, Ar.to(torch.complex64), Bc, Cc, D, z, bias, True)
    y = ops.selective_scan_ref(u, delta, Ar, Bre, Cre, None, None, bias, True,
                               compute_dtype=torch.float64)
    want = (2.0 * y + u.double() * D.double()[:, None]) * F.silu(z.double())
    assert torch.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_complex_scan_brute_force_and_phase_invariance():
    """Brute force on tiny inputs: h_l = sum_{k<=l} exp(A sum_{j=k+1..l}
    delta'_j) delta'_k u_k B_k (a double sum with exponentials of summed
    delta, no recurrence), y_l = 2 Re sum_n h_l C_l + D u. And a phase
    exp(i phi_n) on B with its conjugate on C leaves the output unchanged."""
    for const_b, const_c in ((False, False), (True, False), (False, True)):
        u, delta, A, B, C, D, z, bias = _complex_scan_inputs(b=1, d=2, l=6, n=3, seed=53,
                                                             const_b=const_b, const_c=const_c)
        got = ops.selective_scan_complex_ref(u, delta, A, B, C, D, None, bias, True)
        dl = F.softplus(delta.double() + bias.double()[:, None])
        Bd = ops._bc_complex(B, 1, 2, 6)
        Cd = ops._bc_complex(C, 1, 2, 6)
        A128 = A.to(torch.complex128)
        cs = torch.cumsum(dl, -1)
        want = torch.empty(1, 2, 6, dtype=torch.float64)
        for l in range(6):
            acc = torch.zeros(1, 2, 3, dtype=torch.complex128)
            for k in range(l + 1):
                w = torch.exp(A128[None] * (cs[:, :, l] - cs[:, :, k])[..., None])
                acc = acc + w * (dl[:, :, k] * u[:, :, k].double())[..., None] * Bd[..., k]
            want[:, :, l] = 2.0 * (acc * Cd[..., l]).sum(-1).real + u[:, :, l].double() * D.double()
        assert torch.allclose(got, want, rtol=1e-12, atol=1e-12)
    u, delta, A, B, C, D, z, bias = _complex_scan_inputs(g=2, seed=54)
    phi = torch.rand(6, generator=torch.Generator().manual_seed(3)) * 6.0
    rot = lambda t, s: torch.view_as_real(
        torch.view_as_complex(t.reshape(*t.shape[:-1], -1, 2).contiguous())
        * torch.exp(1j * s * phi.double()).to(torch.complex64)[:, None]).reshape(t.shape)
    base = ops.selective_scan_complex_ref(u, delta, A, B, C, D, z, bias, True)
    turned = ops.selective_scan_complex_ref(u, delta, A, rot(B, 1.0), rot(C, -1.0), D, z, bias, True)
    assert torch.allclose(base, turned, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("const_b,const_c,groups", [(False, False, 1), (False, False, 2),
                                                    (True, True, 1), (True, False, 1)])
def test_complex_scan_bwd_matches_autograd(const_b, const_c, groups):
    """The complex reverse recurrence equals torch autograd of the complex128
    forward oracle (complex gradients packed as dL/dRe + i dL/dIm), every
    gradient, with gate, skip, bias and softplus."""
    u, delta, A, B, C, D, z, bias = _complex_scan_inputs(l=19, g=groups, seed=55 + groups,
                                                         const_b=const_b, const_c=const_c)
    delta = delta - 0.5
    dout = torch.randn(u.shape, generator=torch.Generator().manual_seed(7))
    up = lambda t: (t.to(torch.complex128) if t.is_complex() else t.double()).requires_grad_()
    leaves = [up(t) for t in (u, delta, A, B, C, D, z, bias)]
    out = ops.selective_scan_complex_ref(leaves[0], leaves[1], leaves[2], leaves[3], leaves[4],
                                         leaves[5], leaves[6], leaves[7], True)
    out.backward(dout.double())
    ref = ops.selective_scan_complex_bwd_ref(u, delta, A, B, C, dout, D, z, bias, True)
    for name, r, t in zip("du ddelta dA dB dC dD dz dbias".split(), ref, leaves):
        assert r.shape == t.grad.shape, name
        assert torch.allclose(r, t.grad, rtol=1e-10, atol=1e-11), name


def test_complex_scan_bwd_finite_differences():
    """Central differences of the complex128 forward oracle on a few entries
    of A (real and imaginary parts), of a variable B and C, of delta and u:
    the packed complex gradient is dL/dRe + i dL/dIm."""
    u, delta, A, B, C, D, z, bias = _complex_scan_inputs(b=1, d=2, l=7, n=3, seed=58)
    dout = torch.randn(u.shape, generator=torch.Generator().manual_seed(8))
    ref = ops.selective_scan_complex_bwd_ref(u, delta, A, B, C, dout, D, z, bias, True)
    A128, B64, C64 = A.to(torch.complex128), B.double(), C.double()
    loss = lambda uu, dd, aa, bb, cc: float((ops.selective_scan_complex_ref(
        uu, dd, aa, bb, cc, D, z, bias, True) * dout.double()).sum())
    base = (u.double(), delta.double(), A128, B64, C64)
    eps = 1e-6

    def fd(which, idx, step):
        plus = [t.clone() for t in base]
        minus = [t.clone() for t in base]
        plus[which][idx] += step
        minus[which][idx] -= step
        return (loss(*plus) - loss(*minus)) / (2 * eps)

    for idx in ((0, 0), (1, 2)):
        assert abs(fd(2, idx, eps) - ref[2][idx].real) < 1e-6
        assert abs(fd(2, idx, 1j * eps) - ref[2][idx].imag) < 1e-6
    for idx in ((0, 0, 1, 4), (0, 0, 2, 9)):
        assert abs(fd(3, idx, eps) - ref[3][idx]) < 1e-6
        assert abs(fd(4, idx, eps) - ref[4][idx]) < 1e-6
    for idx in ((0, 0, 3), (0, 1, 6)):
        assert abs(fd(0, idx, eps) - ref[0][idx]) < 1e-6
        assert abs(fd(1, idx, eps) - ref[1][idx]) < 1e-6


def test_complex_chunk_states_pinned():
    """Complex chunk states: the state entry is the complex oracle's last state
    over the prefix; the decay entry is exp(A sum delta') (a product of
    exponentials is the exponential of the sum)."""
    u, delta, A, B, C, D, z, bias = _complex_scan_inputs(l=40, g=2, seed=59)
    xs = ops.selective_scan_complex_chunk_states_ref(u, delta, A, B, bias, True, chunk=16)
    assert xs.shape == (2, 4, 3, 6, 2)
    dl = F.softplus(delta.double() + bias.double()[:, None])
    for k, end in enumerate((16, 32, 40)):
        _, last = ops.selective_scan_complex_ref(u[..., :end], delta[..., :end], A, B[..., :2 * end],
                                                 C[..., :2 * end], None, None, bias, True,
                                                 return_last_state=True)
        assert torch.allclose(xs[:, :, k, :, 1], last, rtol=1e-12, atol=1e-12)
        prod = torch.exp(A.to(torch.complex128)[None] * dl[..., :end].sum(-1)[..., None])
        assert torch.allclose(xs[:, :, k, :, 0], prod, rtol=1e-12, atol=1e-14)


def test_lmhead_ce_ref_softcap_matches_materialised_ce():
    """The streamed lm-head oracle with a logit softcap equals the CE row
    oracle (pinned to F.cross_entropy of the capped logits) on materialised
    logits, for every vocab chunking."""
    g = torch.Generator().manual_seed(17)
    h = torch.randn(40, 32, generator=g)
    W = 2.0 * torch.randn(300, 32, generator=g)
    t = torch.randint(0, 300, (40,), generator=g)
    t[:3] = -100
    logits = h @ W.t()
    per, lse, _, _ = ops.ce_rows_ref(logits, t, softcap=5.0)
    for chunk in (64, 300, 4096):
        loss, lse2, per2 = ops.lmhead_ce_ref(h, W, t, vocab_chunk=chunk, softcap=5.0)
        assert torch.allclose(lse2, lse, rtol=1e-5, atol=1e-5)
        assert torch.allclose(per2, per, rtol=1e-5, atol=1e-5)
        assert torch.allclose(loss, ops.ce_mean_ref(per, t), rtol=1e-5)
    capped = 5.0 * torch.tanh(logits / 5.0)
    ref = F.cross_entropy(capped, t, ignore_index=-100)
    assert torch.allclose(ops.lmhead_ce_ref(h, W, t, softcap=5.0)[0], ref, rtol=1e-5)


def test_lmhead_ce_ref_label_smoothing_matches_torch():
    """Label smoothing in the streamed lm-head oracle equals PyTorch's own
    F.cross_entropy(label_smoothing=a) (whose smoothing term is a times the
    mean of -log_softmax, i.e. a (lse - mean z)), with and without a softcap,
    for every vocab chunking; a = 1 leaves only the uniform term."""
    g = torch.Generator().manual_seed(23)
    h = torch.randn(48, 32, generator=g, dtype=torch.float64).float()
    W = 1.5 * torch.randn(500, 32, generator=g)
    t = torch.randint(0, 500, (48,), generator=g)
    t[[2, 30]] = -100
    logits = h.double() @ W.double().t()
    for cap in (0.0, 4.0):
        z = cap * torch.tanh(logits / cap) if cap else logits
        for a in (0.1, 0.35, 1.0):
            ref = F.cross_entropy(z, t, ignore_index=-100, label_smoothing=a)
            per_ref = F.cross_entropy(z, t, ignore_index=-100, label_smoothing=a, reduction="none")
            for chunk in (64, 500, 4096):
                loss, _, per = ops.lmhead_ce_ref(h, W, t, vocab_chunk=chunk, softcap=cap,
                                                 label_smoothing=a)
                assert torch.allclose(loss.double(), ref, rtol=1e-5), (cap, a, chunk)
                assert torch.allclose(per.double(), per_ref, rtol=1e-5, atol=1e-5)
            # the CE row oracle agrees on the same materialised logits
            per_rows = ops.ce_rows_ref(logits.float(), t, softcap=cap, label_smoothing=a)[0]
            assert torch.allclose(per_rows.double(), per_ref, rtol=1e-5, atol=1e-5)
