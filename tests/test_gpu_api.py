"""GPU: the drop-in surfaces end to end -- torch.ops.autokernel.* with autograd and
autocast, and autokernel.optimize on a small pre-norm transformer (the
reference's test_tier2_parity.py / test_autokernel_autograd_safety.py
checks: rel 5e-3 forward, grads finite and non-zero on every parameter)."""

import pytest
import torch
import torch.nn as nn

from gpu_util import gpu, need_gpu, say

pytestmark = gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_ops_forward_backward(dtype):
    need_gpu()
    import kernels.hip._torch_ops  # noqa: F401
    g = torch.Generator().manual_seed(0)
    x0 = torch.randn(64, 512, generator=g)
    r0 = torch.randn(64, 512, generator=g)
    w0 = 1 + 0.1 * torch.randn(512, generator=g)
    gy = torch.randn(64, 512, generator=g)
    say("ops fwd/bwd", dtype)
    x = x0.to(dtype).to(DEV).requires_grad_()
    r = r0.to(dtype).to(DEV).requires_grad_()
    w = w0.to(dtype).to(DEV).requires_grad_()
    h, n = torch.ops.autokernel.fused_res_rmsnorm(x, r, w, 1e-6)
    (n.float() * gy.to(DEV)).sum().backward()
    xr = x0.to(dtype).double().requires_grad_()
    rr = r0.to(dtype).double().requires_grad_()
    wr = w0.to(dtype).double().requires_grad_()
    hr = xr + rr
    nr = hr / torch.sqrt(hr.pow(2).mean(-1, keepdim=True) + 1e-6) * wr
    (nr * gy.double()).sum().backward()
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for a, b in ((x.grad, xr.grad), (w.grad, wr.grad)):
        rel = float((a.double().cpu() - b).norm() / b.norm())
        assert rel < tol, rel
    # the plain RMSNorm op: values against the oracle, gradients against
    # float64 autograd of the reference formula
    from oracle import ops
    xa = x0.to(dtype).to(DEV).requires_grad_()
    wa = w0.to(dtype).to(DEV).requires_grad_()
    y = torch.ops.autokernel.rmsnorm(xa, wa, 1e-6)
    assert y.dtype == dtype and y.shape == xa.shape
    want = ops.rmsnorm_f32_ref(x0.to(dtype), w0.to(dtype), 1e-6)  # fp32, rounded once
    ytol = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 1.6e-2}[dtype]  # about 1 ulp
    assert torch.allclose(y.detach().cpu().double(), want.double(), rtol=ytol, atol=ytol)
    (y.float() * gy.to(DEV)).sum().backward()
    xb = x0.to(dtype).double().requires_grad_()
    wb = w0.to(dtype).double().requires_grad_()
    yb = xb / torch.sqrt(xb.pow(2).mean(-1, keepdim=True) + 1e-6) * wb
    (yb * gy.double()).sum().backward()
    for a, b in ((xa.grad, xb.grad), (wa.grad, wb.grad)):
        rel = float((a.double().cpu() - b).norm() / b.norm())
        assert rel < tol, rel


def test_autocast_follows_dtype():
    need_gpu()
    import kernels.hip._torch_ops  # noqa: F401
    x = torch.randn(8, 256, device=DEV)
    w = torch.ones(256, device=DEV)
    say("autocast")
    for dt in (torch.float16, torch.bfloat16):
        with torch.autocast("cuda", dtype=dt):
            assert torch.ops.autokernel.rmsnorm(x, w).dtype == dt
            h, n = torch.ops.autokernel.fused_res_rmsnorm(x, x, w)
            assert h.dtype == dt and n.dtype == dt
    assert torch.ops.autokernel.rmsnorm(x, w).dtype == torch.float32


class RMSNorm(nn.Module):
    def __init__(self, d, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d) + 0.05 * torch.randn(d))
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype) * self.weight


class Attn(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.wq = nn.Linear(d, d, bias=False)

    def forward(self, x, freqs_cis):
        return self.wq(x)


class Block(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.attention = Attn(d)
        self.attention_norm = RMSNorm(d)
        self.feed_forward = nn.Sequential(nn.Linear(d, 4 * d, bias=False), nn.SiLU(),
                                          nn.Linear(4 * d, d, bias=False))
        self.ffn_norm = RMSNorm(d)

    def forward(self, x, freqs_cis):
        h = x + self.attention(self.attention_norm(x), freqs_cis)
        return h + self.feed_forward(self.ffn_norm(h))


class TinyLM(nn.Module):
    def __init__(self, d=256, n=3, vocab=1000):
        super().__init__()
        self.emb = nn.Embedding(vocab, d)
        self.layers = nn.ModuleList([Block(d) for _ in range(n)])
        self.norm = RMSNorm(d)
        self.out = nn.Linear(d, vocab, bias=False)

    def forward(self, tok):
        x = self.emb(tok)
        for b in self.layers:
            x = b(x, None)
        return self.out(self.norm(x))


def test_optimize_training_step_bf16():
    need_gpu()
    import autokernel
    torch.manual_seed(0)
    model = TinyLM().to(DEV)
    tok = torch.randint(0, 1000, (4, 64), device=DEV)
    say("optimize tiny LM")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        ref = model(tok).float()
    model = autokernel.optimize(model, training=True)
    rep = autokernel.report(model)
    assert rep["patterns"]["fused_residual_rmsnorm"]["modules_replaced"] == 3
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = model(tok).float()
    rel = float((out - ref).norm() / ref.norm())
    assert rel < 3e-2, rel  # bf16 residual stream through 3 blocks vs the fp32 one
    loss = nn.functional.cross_entropy(out.view(-1, 1000), tok.view(-1))
    loss.backward()
    for name, p in model.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all() and p.grad.abs().sum() > 0, name
