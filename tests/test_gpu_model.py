"""Model-level check on the GPU: one training step of a small pre-norm
transformer with and without ``autokernel.optimize(training=True)``.

Follows the reference's end-to-end checks (verify.py:809-900
``OptimizedModelContext``; scripts/test_autokernel_autograd_safety.py: every
trainable parameter gets a finite, non-zero gradient). The optimized model
runs the gfx950 kernels for RMSNorm, the fused residual + RMSNorm blocks
(forward and backward) and the lm-head + cross-entropy (forward and
backward); the reference model is the same module tree in plain PyTorch.
Bars: loss within 1e-2 relative, each parameter gradient within 3e-2
relative (Frobenius norm), as the reference's chunked-CE and tier-2 parity
scripts allow for bf16 (test_chunked_ce.py:89-90, test_tier2_parity.py:38).
"""

import copy

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from gpu_util import gpu, need_gpu, say

pytestmark = gpu
DEV = "cuda"


class RMSNorm(nn.Module):
    def __init__(self, d, eps=1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype) * self.weight


class Mixer(nn.Module):
    """Causal token mixing without batched matmuls: a running mean over the
    sequence, then a projection (stands in for attention)."""

    def __init__(self, d):
        super().__init__()
        self.wv = nn.Linear(d, d, bias=False)
        self.wo = nn.Linear(d, d, bias=False)

    def forward(self, x, freqs_cis):
        v = self.wv(x).float()
        n = torch.arange(1, x.shape[1] + 1, device=x.device, dtype=torch.float32)[None, :, None]
        return self.wo((v.cumsum(1) / n).to(x.dtype))


class FeedForward(nn.Module):
    def __init__(self, d, hidden):
        super().__init__()
        self.w1 = nn.Linear(d, hidden, bias=False)
        self.w2 = nn.Linear(hidden, d, bias=False)
        self.w3 = nn.Linear(d, hidden, bias=False)

    def forward(self, x):
        return self.w2(F.silu(self.w1(x)) * self.w3(x))


class Block(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.attention = Mixer(d)
        self.attention_norm = RMSNorm(d)
        self.feed_forward = FeedForward(d, 4 * d)
        self.ffn_norm = RMSNorm(d)

    def forward(self, x, freqs_cis):
        h = x + self.attention(self.attention_norm(x), freqs_cis)
        return h + self.feed_forward(self.ffn_norm(h))


class TinyLM(nn.Module):
    def __init__(self, vocab=2048, d=256, n_layers=3):
        super().__init__()
        self.tok_embeddings = nn.Embedding(vocab, d)
        self.layers = nn.ModuleList([Block(d) for _ in range(n_layers)])
        self.norm = RMSNorm(d)
        self.output = nn.Linear(d, vocab, bias=False)

    def hidden(self, tokens):
        x = self.tok_embeddings(tokens)
        for layer in self.layers:
            x = layer(x, None)
        return self.norm(x)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_optimized_training_step_matches_pytorch(dtype):
    need_gpu()
    import autokernel
    from kernels.hip.chunked_linear_cross_entropy import ChunkedLinearCrossEntropyLoss
    torch.manual_seed(0)
    ref = TinyLM().to(DEV, dtype)
    opt = autokernel.optimize(copy.deepcopy(ref), dtype=dtype, training=True)
    report = autokernel.report(opt)
    say("model-level training step", dtype, report)
    names = {type(m).__name__ for m in opt.modules()}
    assert "_FusedResidualRMSNormBlockReplacement" in names and "_RMSNormReplacement" in names

    g = torch.Generator().manual_seed(1)
    tokens = torch.randint(0, 2048, (4, 128), generator=g).to(DEV)
    targets = torch.randint(0, 2048, (4, 128), generator=g)
    targets[0, :16] = -100
    targets = targets.to(DEV)

    h = ref.hidden(tokens)
    loss_ref = F.cross_entropy(ref.output(h).float().reshape(-1, 2048), targets.reshape(-1))
    loss_ref.backward()
    ho = opt.hidden(tokens)
    loss_opt = ChunkedLinearCrossEntropyLoss()(ho, opt.output.weight, targets)
    loss_opt.backward()

    assert abs(float(loss_opt) - float(loss_ref)) <= 1e-2 * abs(float(loss_ref))
    ref_grads = dict(ref.named_parameters())
    opt_grads = {}
    for name, p in opt.named_parameters():
        opt_grads[name] = p
    # the block replacement keeps the submodules and renames ffn_norm.weight
    # to ffn_norm_weight (the reference replacement's state-dict key)
    checked = 0
    for name, p in ref_grads.items():
        oname = name.replace("ffn_norm.weight", "ffn_norm_weight")
        q = opt_grads[oname]
        assert q.grad is not None and torch.isfinite(q.grad).all(), name
        assert float(q.grad.float().abs().sum()) > 0, name
        rel = float((q.grad.float() - p.grad.float()).norm() / p.grad.float().norm())
        assert rel < 3e-2, (name, rel)
        checked += 1
    assert checked == len(ref_grads)
