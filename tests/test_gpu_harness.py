"""GPU: the staged correctness + timing harness (harness.py, the reference's
bench.py KERNEL_CONFIGS / run_correctness / FINAL lines) for every kernel type
of the set, through ``bench.py --harness``, and the model verifier
(verify.OptimizedModelContext) on a pre-norm LM with the gfx950 kernels
swapped in.

Bars: the harness's own (the reference harness's tolerances against eager
PyTorch evaluating reference.py in fp32, the five adversarial transforms,
bitwise determinism, edge sizes) -- every stage must PASS; the model output
within the verifier's dtype tolerance of the unmodified model.
"""

import os
import subprocess
import sys

import pytest
import torch

from gpu_util import gpu, need_gpu, say

pytestmark = gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("kernel_type", ["softmax", "cross_entropy", "rmsnorm",
                                         "fused_residual_add_rmsnorm", "selective_scan"])
def test_harness_all_stages_pass(kernel_type):
    need_gpu()
    import harness
    say("harness", kernel_type)
    lines = []
    out = harness.main(["--kernel", kernel_type, "--sizes", "small", "--reps", "20"], log=lines.append)
    corr = out["correctness"]
    assert corr["correctness"] == "PASS", corr.get("details")
    for stage in ("smoke_test", "shape_sweep", "determinism", "edge_cases"):
        assert corr[stage].startswith("PASS"), (stage, corr[stage])
    assert corr["numerical_stability"].startswith("PASS" if kernel_type != "selective_scan" else "SKIP")
    text = "\n".join(lines)
    final = text[text.index("=== FINAL ==="):]
    for key in ("kernel_type: " + kernel_type, "correctness: PASS", "throughput_tflops:",
                "speedup_vs_pytorch:", "pct_peak_compute:", "bench_time_seconds:"):
        assert key in final, key
    assert out["performance"]["primary"]["kernel_latency_us"] > 0


def test_bench_py_harness_mode_prints_final_lines():
    """``python bench.py --harness rmsnorm --quick`` in its own process."""
    need_gpu()
    say("bench.py --harness")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--harness", "rmsnorm", "--quick"],
                       capture_output=True, text=True, timeout=240, cwd=ROOT)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "=== FINAL ===" in r.stdout and "correctness: PASS" in r.stdout


def test_optimized_model_context_on_a_prenorm_lm():
    """A LLaMA-style pre-norm LM in bf16 with its RMSNorms and blocks swapped
    for the gfx950 kernels inside the context; output within the bf16
    tolerance of the unmodified model, originals restored afterwards."""
    need_gpu()
    import torch.nn as nn
    import torch.nn.functional as F
    import verify

    class RMSNorm(nn.Module):
        def __init__(self, d, eps=1e-5):
            super().__init__()
            self.weight = nn.Parameter(torch.ones(d))
            self.eps = eps

        def forward(self, x):
            xf = x.float()
            return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype) * self.weight

    class Attention(nn.Module):
        def __init__(self, d, h):
            super().__init__()
            self.h = h
            self.wqkv = nn.Linear(d, 3 * d, bias=False)
            self.wo = nn.Linear(d, d, bias=False)

        def forward(self, x, freqs_cis):
            B, T, D = x.shape
            q, k, v = self.wqkv(x).view(B, T, 3, self.h, D // self.h).unbind(2)
            y = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                               is_causal=True)
            return self.wo(y.transpose(1, 2).reshape(B, T, D))

    class FeedForward(nn.Module):
        def __init__(self, d):
            super().__init__()
            self.w1 = nn.Linear(d, 4 * d, bias=False)
            self.w2 = nn.Linear(4 * d, d, bias=False)

        def forward(self, x):
            return self.w2(F.gelu(self.w1(x)))

    class Block(nn.Module):
        def __init__(self, d, h):
            super().__init__()
            self.attention = Attention(d, h)
            self.attention_norm = RMSNorm(d)
            self.feed_forward = FeedForward(d)
            self.ffn_norm = RMSNorm(d)

        def forward(self, x, freqs_cis):
            h = x + self.attention(self.attention_norm(x), freqs_cis)
            return h + self.feed_forward(self.ffn_norm(h))

    class LM(nn.Module):
        def __init__(self, vocab=1000, d=256, h=4, n=3):
            super().__init__()
            self.tok = nn.Embedding(vocab, d)
            self.layers = nn.ModuleList([Block(d, h) for _ in range(n)])
            self.norm = RMSNorm(d)
            self.out = nn.Linear(d, vocab, bias=False)

        def forward(self, idx):
            x = self.tok(idx)
            for layer in self.layers:
                x = layer(x, None)
            return self.out(self.norm(x))

    torch.manual_seed(0)
    model = LM().cuda().to(torch.bfloat16)
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, RMSNorm):
                m.weight.add_(0.05 * torch.randn_like(m.weight))
    idx = torch.randint(0, 1000, (4, 128), device="cuda")
    say("verify_model prenorm LM")
    reps = [verify.KernelReplacement("fused_residual_add_rmsnorm", rank=0, speedup=6.6),
            verify.KernelReplacement("rmsnorm", rank=1, speedup=3.3)]
    res = verify.verify_model(model, (idx,), reps, torch.bfloat16, atol=0.1, rtol=0.05)
    assert res.correctness == "PASS", res.comparison.get("reason")
    assert len(res.kernels_replaced) == 2 and res.opt_latency_ms > 0
    assert all(type(m).__name__ in ("Block", "RMSNorm") for m in model.modules()
               if "Norm" in type(m).__name__ or "Block" in type(m).__name__)
