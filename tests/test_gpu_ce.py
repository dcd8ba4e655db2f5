"""GPU parity: cross-entropy over materialised logits (kernels/ce_fused.py API).

Bars: per-row loss and logsumexp within 1e-4 relative (+1e-5 absolute) of the
fp32 oracle on the same rounded logits; the mean loss within 1e-3 relative
of float64 F.cross_entropy (north-star CE bar); gradients within 1 ulp of the
logits dtype plus 1e-6 absolute; ignore-index handling exact.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from gpu_util import gpu, need_gpu, say
from oracle import ops

pytestmark = gpu
DEV = "cuda"


def _close(a, b, rtol=1e-4, atol=1e-5):
    return torch.allclose(a.double().cpu(), b.double().cpu(), rtol=rtol, atol=atol)


def _grad_ok(g, ref, dtype):
    ulp = {torch.float32: 2 ** -23, torch.float16: 2 ** -10, torch.bfloat16: 2 ** -7}[dtype]
    d = (g.float().cpu() - ref.float()).abs()
    return bool((d <= ref.float().abs() * ulp * 2 + 1e-6).all()), float(d.max())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("vocab", [1000, 32768, 50257, 50304])
@pytest.mark.parametrize("softcap,ls", [(0.0, 0.0), (30.0, 0.0), (0.0, 0.1), (15.0, 0.05)])
def test_ce_fwd_matches_oracle(dtype, vocab, softcap, ls):
    need_gpu()
    from kernels.ce_fused import _get_fwd_module
    g = torch.Generator().manual_seed(vocab)
    B = 64
    logits = (3 * torch.randn(B, vocab, generator=g)).to(dtype)
    t = torch.randint(0, vocab, (B,), generator=g)
    t[[0, 5, 63]] = -100
    say("ce_fwd", dtype, vocab, softcap, ls)
    losses, lse, mx, sm, grad = _get_fwd_module().cross_entropy_fwd_hip(
        logits.to(DEV), t.to(DEV), softcap, -100, ls, 1, 1, 1.0 / 61)
    rl, rlse, rmx, rsm = ops.ce_rows_ref(logits, t, softcap, -100, ls)
    assert _close(losses, rl) and _close(lse, rlse)
    assert _close(mx, rmx, rtol=0, atol=0) or _close(mx, rmx, rtol=1e-6, atol=1e-6)
    assert _close(sm, rsm, rtol=1e-4)
    assert float(losses[0]) == 0.0 and float(losses[63]) == 0.0
    gref = ops.ce_grad_ref(logits, t, softcap, -100, ls, 1.0 / 61)
    ok, worst = _grad_ok(grad, gref, dtype)
    assert ok, worst
    assert bool((grad[[0, 5, 63]] == 0).all())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_ce_bwd_tiny_matches_oracle(dtype):
    need_gpu()
    from kernels.ce_fused import _get_bwd_module, _get_fwd_module
    g = torch.Generator().manual_seed(3)
    logits = (2 * torch.randn(48, 4099, generator=g)).to(dtype)
    t = torch.randint(0, 4099, (48,), generator=g)
    t[7] = -100
    say("ce_bwd_tiny", dtype)
    _, _, mx, sm, _ = _get_fwd_module().cross_entropy_fwd_hip(logits.to(DEV), t.to(DEV), 20.0, -100, 0.1, 0, 1, 1.0)
    grad = _get_bwd_module().cross_entropy_bwd_tiny_hip(logits.to(DEV), t.to(DEV), mx, sm, 20.0, -100, 0.1, 0.25)
    ok, worst = _grad_ok(grad, ops.ce_grad_ref(logits, t, 20.0, -100, 0.1, 0.25), dtype)
    assert ok, worst


@pytest.mark.parametrize("mode", ["fused", "tiny"])
def test_ce_full_and_kernel_fn_vs_torch(mode):
    need_gpu()
    from kernels.ce_fused import ce_full, kernel_fn
    g = torch.Generator().manual_seed(4)
    base = (3 * torch.randn(256, 32768, generator=g)).half()
    t = torch.randint(0, 32768, (256,), generator=g)
    t[torch.randperm(256, generator=g)[:12]] = -100
    say("ce_full", mode)
    ref = F.cross_entropy(base.double(), t)
    loss = kernel_fn(base.to(DEV), t.to(DEV))
    assert abs(float(loss) - float(ref)) <= 1e-3 * abs(float(ref))
    x = base.to(DEV).requires_grad_()
    l2, lse = ce_full(x, t.to(DEV), mode=mode, return_z=True, z_loss_weight=1e-4 if mode == "tiny" else 0.0)
    l2.backward()
    xr = base.double().requires_grad_()
    r2 = F.cross_entropy(xr, t)
    if mode == "tiny":
        valid = (t != -100).double()
        r2 = r2 + 1e-4 * ((torch.logsumexp(xr, -1) * valid) ** 2).sum() / valid.sum()
    r2.backward()
    assert abs(float(l2) - float(r2)) <= 1e-3 * abs(float(r2))
    gd = (x.grad.double().cpu() - xr.grad).abs().max()
    assert float(gd) < 5e-6, float(gd)   # half an fp16 ulp at |g| ~ 4e-3 is 1.9e-6
    assert _close(lse, torch.logsumexp(base.double(), -1), rtol=1e-5)


def test_ce_out_of_range_target_is_nan_not_oob():
    need_gpu()
    from kernels.ce_fused import _get_fwd_module
    logits = torch.randn(4, 100).half().to(DEV)
    t = torch.tensor([1, 100, -5, -100]).to(DEV)
    say("ce bad targets")
    losses, lse, _, _, grad = _get_fwd_module().cross_entropy_fwd_hip(logits, t, 0.0, -100, 0.0, 1, 0, 1.0)
    lc = losses.cpu()
    assert math.isfinite(float(lc[0])) and math.isnan(float(lc[1])) and math.isnan(float(lc[2]))
    assert float(lc[3]) == 0.0 and bool((grad[3] == 0).all())


@pytest.mark.parametrize("mode", ["fused", "tiny"])
@pytest.mark.parametrize("softcap,ls", [(0.0, 0.0), (12.0, 0.1)])
def test_ce_zloss_in_kernel_vs_float64_autograd(mode, softcap, ls):
    """The z-loss gradient 2 w lse p comes from the CE kernels themselves, in
    either mode and through the softcap; the loss and lse from ak_ce_mean.
    Bars: loss 1e-3 relative (the CE bar), gradient within 1 bf16 ulp of its
    magnitude plus 1e-6."""
    need_gpu()
    from kernels.ce_fused import ce_full
    g = torch.Generator().manual_seed(21)
    base = (4 * torch.randn(96, 5003, generator=g)).bfloat16()
    t = torch.randint(0, 5003, (96,), generator=g)
    t[torch.randperm(96, generator=g)[:9]] = -100
    w = 2e-3
    say("ce z-loss", mode, softcap, ls)
    x = base.to(DEV).requires_grad_()
    loss, lse = ce_full(x, t.to(DEV), softcap=softcap, label_smoothing=ls, mode=mode,
                        return_z=True, z_loss_weight=w)
    (3.0 * loss).backward()
    xr = base.double().requires_grad_()
    xc = softcap * torch.tanh(xr / softcap) if softcap > 0 else xr
    valid = (t != -100).double()
    ref = F.cross_entropy(xc, t, label_smoothing=ls) + w * (
        (torch.logsumexp(xc, -1) ** 2) * valid).sum() / valid.sum()
    (3.0 * ref).backward()
    assert abs(float(loss) - float(ref)) <= 1e-3 * abs(float(ref))
    assert _close(lse, torch.logsumexp(xc.detach(), -1), rtol=1e-5)
    ok, worst = _grad_ok(x.grad, xr.grad, torch.bfloat16)
    assert ok, worst
    assert bool((x.grad[t.to(DEV) == -100] == 0).all())


def test_ce_count_and_mean_many_rows():
    """ak_ce_count_valid / ak_ce_mean over 300k rows against the oracle; the
    count is exact, the mean within 1e-5 relative (fp32 sums), deterministic."""
    need_gpu()
    from kernels.hip import _lib
    g = torch.Generator().manual_seed(22)
    n = 300_001
    losses = torch.rand(n, generator=g) * 5
    lse = torch.randn(n, generator=g) * 3
    t = torch.randint(0, 1000, (n,), generator=g)
    t[torch.randperm(n, generator=g)[:12345]] = -7
    say("ce count/mean", n)
    tg = t.to(DEV)
    denom = _lib.ce_count_valid(tg, -7).cpu()
    nv = n - 12345
    assert float(denom[0]) == float(nv) and float(denom[1]) == float(torch.tensor(1.0 / nv))
    cnt = torch.empty(1, dtype=torch.int64, device=DEV)
    m1 = _lib.ce_mean(losses.to(DEV), lse.to(DEV), tg, -7, 0.01, n_valid=cnt)
    m2 = _lib.ce_mean(losses.to(DEV), lse.to(DEV), tg, -7, 0.01)
    ref = ops.ce_mean_ref(losses.double(), t, -7, lse.double(), 0.01)
    assert int(cnt) == nv
    assert abs(float(m1) - float(ref)) <= 1e-5 * abs(float(ref))
    assert torch.equal(m1, m2)
    all_ignored = torch.full((10,), -7, device=DEV)
    assert float(_lib.ce_count_valid(all_ignored, -7)[0]) == 1.0
    assert float(_lib.ce_mean(torch.ones(10, device=DEV), None, all_ignored, -7)) == 0.0


@pytest.mark.parametrize("up", [1.0, 0.7])
def test_ce_fused_backward_scales_on_device(up):
    """Fused mode: the backward applies the upstream gradient on the device
    (torch's sync debug mode set to error around it). An upstream gradient
    of 1 returns the gradient the forward wrote, bit for bit; 0.7 the same
    gradient times bf16(0.7), rounded once."""
    need_gpu()
    from kernels.ce_fused import ce_full
    g = torch.Generator().manual_seed(33)
    base = (2 * torch.randn(64, 3001, generator=g)).bfloat16()
    t = torch.randint(0, 3001, (64,), generator=g)
    t[5] = -100
    say("ce fused backward on device", up)
    x = base.to(DEV).requires_grad_()
    loss = ce_full(x, t.to(DEV), mode="fused")
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        (up * loss).backward()
    finally:
        torch.cuda.set_sync_debug_mode("default")
    # the forward's own gradient: the same kernel call the fused forward makes
    from kernels.hip import _lib
    td = t.to(DEV)
    denom = _lib.ce_count_valid(td, -100)
    gref = torch.empty_like(x)
    f32 = dict(dtype=torch.float32, device=DEV)
    _lib.ce_fwd(base.to(DEV), td, torch.empty(64, **f32), torch.empty(64, **f32), None, None, gref,
                0.0, -100, 0.0, 1.0, scale_dev=denom[1:])
    want = gref if up == 1.0 else gref * torch.tensor(up, device=DEV).bfloat16()
    assert torch.equal(x.grad, want)
