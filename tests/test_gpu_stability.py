"""GPU numerical stability under the reference harness's adversarial inputs.

The reference's kernel harness (bench.py:1205-1213) re-runs each kernel on
five transforms of its inputs: near_max (x 60000 for fp16, x 1e30 otherwise),
near_zero (x 1e-6), mixed_scale (each element x 1e3 or x 1e-3), all_zeros and
all_same (0.5). It accepts NaN / Inf only where the reference output has them
too, and otherwise compares at 10x relaxed tolerances (:1228-1250).

Bars here are stricter: the non-finite pattern (NaN and +/-Inf, element by
element) must equal the oracle's, and the finite entries meet the usual bars
(norm and softmax within 1 ulp of the oracle's fp32-computed value, fp32
within 1e-5 relative, new_residual bit-exact, CE loss within 1e-3 relative).
"""

import pytest
import torch

from gpu_util import gpu, max_ulp, need_gpu, say
from oracle import ops

pytestmark = gpu
DEV = "cuda"

TRANSFORMS = ("near_max", "near_zero", "mixed_scale", "all_zeros", "all_same")


def _transform(name, t, g):
    """The reference harness's transforms, applied in t's dtype."""
    if name == "near_max":
        return t * 60000.0 if t.dtype == torch.float16 else t * 1e30
    if name == "near_zero":
        return t * 1e-6
    if name == "mixed_scale":
        pick = torch.rand(t.shape, generator=g).to(t.dtype) > 0.5
        return t * torch.where(pick, torch.tensor(1e3, dtype=t.dtype), torch.tensor(1e-3, dtype=t.dtype))
    if name == "all_zeros":
        return torch.zeros_like(t)
    return torch.ones_like(t) * 0.5


def _same_nonfinite(a, b):
    a, b = a.cpu(), b.cpu()
    return torch.equal(torch.isnan(a), torch.isnan(b)) and torch.equal(a == float("inf"), b == float("inf")) \
        and torch.equal(a == float("-inf"), b == float("-inf"))


def _finite_close(y, ref):
    """Finite entries: 1 ulp for fp16 / bf16, 1e-5 relative (+1e-7 of the row scale) for fp32."""
    y, ref = y.cpu(), ref.cpu()
    m = torch.isfinite(ref)
    if not bool(m.any()):
        return True
    if y.dtype == torch.float32:
        d = (y[m].double() - ref[m].double()).abs()
        return bool((d <= 1e-5 * ref[m].double().abs() + 1e-7 * ref[m].double().abs().max()).all())
    return max_ulp(y[m], ref[m]) <= 1


def _check(y, ref, what):
    assert _same_nonfinite(y, ref), f"{what}: NaN/Inf pattern differs from the oracle"
    assert _finite_close(y, ref), f"{what}: finite entries off the oracle"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", TRANSFORMS)
def test_softmax_adversarial(dtype, case):
    need_gpu()
    from kernels.hip import softmax
    g = torch.Generator().manual_seed(42)
    x = _transform(case, (3 * torch.randn(48, 1000, generator=g)).to(dtype), g)
    say("softmax adversarial", case, dtype)
    _check(softmax.kernel_fn(x.to(DEV)), ops.softmax_ref(x), f"softmax {case} {dtype}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", TRANSFORMS)
def test_rmsnorm_adversarial(dtype, case):
    need_gpu()
    from kernels.hip import rmsnorm
    g = torch.Generator().manual_seed(42)
    x = _transform(case, torch.randn(32, 1024, generator=g).to(dtype), g)
    w = _transform(case, (1 + 0.02 * torch.randn(1024, generator=g)).to(dtype), g)
    say("rmsnorm adversarial", case, dtype)
    y = rmsnorm.kernel_fn(x.to(DEV), w.to(DEV))
    ref = ops.rmsnorm_f32_ref(x, w) if dtype != torch.float32 else ops.rmsnorm_ref(x, w)
    _check(y, ref, f"rmsnorm {case} {dtype}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", TRANSFORMS)
def test_fused_add_rmsnorm_adversarial(dtype, case):
    need_gpu()
    from kernels.hip import fused_residual_add_rmsnorm as frn
    g = torch.Generator().manual_seed(42)
    x = _transform(case, torch.randn(32, 2048, generator=g).to(dtype), g)
    r = _transform(case, torch.randn(32, 2048, generator=g).to(dtype), g)
    w = _transform(case, (1 + 0.02 * torch.randn(2048, generator=g)).to(dtype), g)
    say("fused add+rmsnorm adversarial", case, dtype)
    h, y = frn.kernel_fn_dual(x.to(DEV), r.to(DEV), w.to(DEV))
    href, yref = ops.fused_residual_add_rmsnorm_ref(x, r, w)
    h = h.cpu()
    assert _same_nonfinite(h, href)
    ok = ~torch.isnan(href)
    assert torch.equal(h[ok], href[ok]), f"new_residual {case} {dtype} not bit-exact"
    _check(y, yref, f"fused add+rmsnorm {case} {dtype}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", TRANSFORMS)
def test_cross_entropy_adversarial(dtype, case):
    need_gpu()
    from kernels.ce_fused import kernel_fn
    g = torch.Generator().manual_seed(42)
    logits = _transform(case, torch.randn(64, 5000, generator=g).to(dtype), g)
    t = torch.randint(0, 5000, (64,), generator=g)
    t[:4] = -100
    say("cross entropy adversarial", case, dtype)
    loss = float(kernel_fn(logits.to(DEV), t.to(DEV)))
    per, _, _, _ = ops.ce_rows_ref(logits, t)
    ref = float(ops.ce_mean_ref(per, t))
    if ref != ref or abs(ref) == float("inf"):
        assert loss != loss or abs(loss) == float("inf"), (case, loss, ref)
    else:
        assert abs(loss - ref) <= 1e-3 * abs(ref) + 1e-6, (case, loss, ref)
