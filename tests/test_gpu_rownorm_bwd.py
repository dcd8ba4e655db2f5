"""GPU parity: RMSNorm backward and fused residual + RMSNorm backward.

Against the float64 oracle (``oracle.ops.rmsnorm_bwd_ref``, pinned to torch
autograd in tests/test_oracle.py). Bars:
* grad_x: within 1 ulp of the element type of the exact value, plus an fp32
  arithmetic allowance of 2e-6 of the row's largest term
  r * (|g_j w_j| + |n_j| |c|) (the kernel computes in fp32 and rounds once);
* grad_weight (fp32, a sum over rows): within 1e-5 of sum_rows |dy * n| per
  column;
* grad_weight bitwise identical across runs (fixed summation order).
"""

import pytest
import torch

from gpu_util import gpu, need_gpu, say
from oracle import ops

pytestmark = gpu
DEV = "cuda"

_MANT = {torch.float32: 23, torch.float16: 10, torch.bfloat16: 7}


def _ulp(ref64: torch.Tensor, dtype) -> torch.Tensor:
    """Spacing of dtype's grid at |ref| (normal range; fp16 subnormals floor at 2^-24)."""
    _, e = torch.frexp(ref64.abs().clamp_min(1e-30))
    u = torch.ldexp(torch.ones_like(ref64), (e - 1 - _MANT[dtype]).to(torch.int32))
    if dtype == torch.float16:
        u = u.clamp_min(2.0 ** -24)
    return u


def _check_gx(gx, x, w, dy, dh, eps):
    xd, wd, gd = x.double().cpu(), w.double().cpu(), dy.double().cpu()
    ref, _ = ops.rmsnorm_bwd_ref(x.cpu(), w.cpu(), dy.cpu(), eps)
    if dh is not None:
        ref = ref + dh.double().cpu()
    r = 1.0 / torch.sqrt((xd * xd).mean(-1, keepdim=True) + eps)
    n = xd * r
    g = gd * wd
    c = (g * n).mean(-1, keepdim=True)
    scale = (r * (g.abs() + n.abs() * c.abs())).amax(-1, keepdim=True)
    if dh is not None:
        scale = scale + dh.double().cpu().abs().amax(-1, keepdim=True)
    bound = _ulp(ref, gx.dtype) + 2e-6 * scale
    err = (gx.double().cpu() - ref).abs()
    assert bool((err <= bound).all()), float((err / bound).max())


def _check_gw(gw, x, w, dy, eps):
    _, ref = ops.rmsnorm_bwd_ref(x.cpu(), w.cpu(), dy.cpu(), eps)
    xd = x.double().cpu().reshape(-1, x.shape[-1])
    r = 1.0 / torch.sqrt((xd * xd).mean(-1, keepdim=True) + eps)
    mag = (dy.double().cpu().reshape(-1, x.shape[-1]) * xd * r).abs().sum(0)
    err = (gw.double().cpu() - ref).abs()
    assert bool((err <= 1e-5 * mag + 1e-30).all()), float((err / (mag + 1e-30)).max())


def _inputs(rows, cols, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = (2 * torch.randn(rows, cols, generator=g)).to(dtype)
    w = (1 + 0.1 * torch.randn(cols, generator=g)).to(dtype)
    dy = torch.randn(rows, cols, generator=g).to(dtype)
    dh = torch.randn(rows, cols, generator=g).to(dtype)
    return x, w, dy, dh


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,cols", [
    (3000, 64), (1100, 256), (600, 768), (700, 1000), (37, 4096), (530, 4104), (9, 16384),
    (5, 65536), (33, 7), (5, 70000), (1, 512), (2, 4096)])
def test_rmsnorm_bwd_shapes(dtype, rows, cols):
    need_gpu()
    from kernels.hip import rmsnorm_backward as rb
    x, w, dy, _ = _inputs(rows, cols, dtype, rows * 7 + cols)
    say("rmsnorm bwd", rows, cols, dtype)
    gx, gw = rb.kernel_fn(x.to(DEV), w.to(DEV), dy.to(DEV), eps=1e-6)
    assert gx.dtype == dtype and gw.dtype == torch.float32
    _check_gx(gx, x, w, dy, None, 1e-6)
    _check_gw(gw, x, w, dy, 1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,cols", [(3000, 64), (600, 768), (37, 4096), (9, 16384), (33, 7)])
@pytest.mark.parametrize("with_dh", [True, False])
def test_fused_bwd_shapes(dtype, rows, cols, with_dh):
    need_gpu()
    from kernels.hip import fused_residual_rmsnorm_backward as frb
    h, w, gn, gh = _inputs(rows, cols, dtype, rows + 3 * cols)
    say("fused rmsnorm bwd", rows, cols, dtype, with_dh)
    ghd = gh.to(DEV) if with_dh else None
    gx, gr, gw = frb.kernel_fn(h.to(DEV), w.to(DEV), ghd, gn.to(DEV), eps=1e-5)
    assert gx is gr and gx.dtype == dtype
    _check_gx(gx, h, w, gn, gh if with_dh else None, 1e-5)
    _check_gw(gw, h, w, gn, 1e-5)


def test_strided_rows_generic_and_vector_paths():
    """Row pitches that keep (multiple of 8) and break (odd) the vector path."""
    need_gpu()
    from kernels.hip import _lib
    for pitch in (1032, 1025):
        x, w, dy, _ = _inputs(64, 1024, torch.bfloat16, pitch)
        say("rmsnorm bwd pitch", pitch)
        xb = torch.zeros(64, pitch, dtype=torch.bfloat16, device=DEV)
        gb = torch.zeros(64, pitch, dtype=torch.bfloat16, device=DEV)
        ob = torch.full((64, pitch), 7.0, dtype=torch.bfloat16, device=DEV)
        xb[:, :1024] = x.to(DEV)
        gb[:, :1024] = dy.to(DEV)
        gw = torch.empty(1024, dtype=torch.float32, device=DEV)
        ws = torch.empty(_lib.rmsnorm_bwd_workspace_bytes(64, 1024), dtype=torch.uint8, device=DEV)
        _lib.rmsnorm_bwd(xb[:, :1024], w.to(DEV), gb[:, :1024], ob[:, :1024], gw, ws, 1e-6)
        _check_gx(ob[:, :1024], x, w, dy, None, 1e-6)
        _check_gw(gw, x, w, dy, 1e-6)
        assert bool((ob[:, 1024:].float().cpu() == 7.0).all())  # padding untouched


def test_no_weight_grad_and_empty_rows():
    need_gpu()
    from kernels.hip import _lib
    x, w, dy, _ = _inputs(40, 512, torch.float16, 1)
    say("rmsnorm bwd without grad_weight; rows = 0")
    gx = torch.empty_like(x, device=DEV)
    _lib.rmsnorm_bwd(x.to(DEV), w.to(DEV), dy.to(DEV), gx, None, None, 1e-6)
    _check_gx(gx, x, w, dy, None, 1e-6)
    gw = torch.full((512,), 3.0, device=DEV)
    e = torch.empty(0, 512, dtype=torch.float16, device=DEV)
    _lib.rmsnorm_bwd(e, w.to(DEV), e, e, gw, None, 1e-6)
    assert torch.equal(gw.cpu(), torch.zeros(512))


def test_weight_grad_deterministic():
    need_gpu()
    from kernels.hip import rmsnorm_backward as rb
    x, w, dy, _ = _inputs(5000, 768, torch.bfloat16, 9)
    say("rmsnorm bwd determinism")
    outs = [rb.kernel_fn(x.to(DEV), w.to(DEV), dy.to(DEV)) for _ in range(3)]
    for gx, gw in outs[1:]:
        assert torch.equal(gx, outs[0][0]) and torch.equal(gw, outs[0][1])


def test_c3_shape_fused_backward():
    """The fused backward at the C3 forward's shape (bf16 [16384, 4096])."""
    need_gpu()
    import bench
    from kernels.hip import fused_residual_rmsnorm_backward as frb
    c = bench.gen_c3()
    g = torch.Generator().manual_seed(1)
    gh = torch.randn(16384, 4096, generator=g).bfloat16()
    gn = torch.randn(16384, 4096, generator=g).bfloat16()
    hidden, _ = ops.fused_residual_add_rmsnorm_ref(c["x"], c["r"], c["w"], c["eps"])
    say("C3-shape fused rmsnorm backward bf16 [16384, 4096]")
    gx, _, gw = frb.kernel_fn(hidden.to(DEV), c["w"].to(DEV), gh.to(DEV), gn.to(DEV), eps=c["eps"])
    for lo in range(0, 16384, 4096):
        sl = slice(lo, lo + 4096)
        _check_gx(gx[sl], hidden[sl], c["w"], gn[sl], gh[sl], c["eps"])
    _check_gw(gw, hidden, c["w"], gn, c["eps"])


def test_c3_shape_fused_backward_homogeneous_bitwise():
    """Full C3 shape: grad_x and grad_weight are linear in the upstream
    gradients and doubling both is exact through the row sums, the fixed-order
    column sums and the final rounding: grads(2 gh, 2 gn) == 2 grads(gh, gn)."""
    need_gpu()
    import bench
    from kernels.hip import fused_residual_rmsnorm_backward as frb
    c = bench.gen_c3()
    g = torch.Generator().manual_seed(2)
    gh = torch.randn(16384, 4096, generator=g).bfloat16().to(DEV)
    gn = torch.randn(16384, 4096, generator=g).bfloat16().to(DEV)
    hidden, _ = ops.fused_residual_add_rmsnorm_ref(c["x"], c["r"], c["w"], c["eps"])
    hidden, w = hidden.to(DEV), c["w"].to(DEV)
    say("C3-shape fused backward homogeneity")
    gx1, _, gw1 = frb.kernel_fn(hidden, w, gh, gn, eps=c["eps"])
    gx2, _, gw2 = frb.kernel_fn(hidden, w, 2 * gh, 2 * gn, eps=c["eps"])
    assert torch.equal(gx2, 2 * gx1) and torch.equal(gw2, 2 * gw1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_custom_op_autograd_uses_kernels(dtype):
    """torch.ops.autokernel.{rmsnorm, fused_res_rmsnorm} backward on the GPU
    (the gfx950 backward kernels) against float64 autograd of the oracle."""
    need_gpu()
    import kernels.hip._torch_ops as T
    assert T._bwd_kernels_for(torch.empty(1, device=DEV))
    g = torch.Generator().manual_seed(4)
    x = torch.randn(64, 768, generator=g).to(dtype)
    r = torch.randn(64, 768, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(768, generator=g)).to(dtype)
    up = torch.randn(64, 768, generator=g).to(dtype)
    say("custom op autograd", dtype)
    xd, wd = x.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
    torch.ops.autokernel.rmsnorm(xd, wd, 1e-6).backward(up.to(DEV))
    x64, w64 = x.double().requires_grad_(), w.double().requires_grad_()
    ops.rmsnorm_ref(x64, w64, 1e-6).backward(up.double())
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert torch.allclose(xd.grad.double().cpu(), x64.grad, rtol=tol, atol=tol)
    assert torch.allclose(wd.grad.double().cpu(), w64.grad, rtol=tol, atol=tol * 64)
    xd, rd_, wd = (t.to(DEV).requires_grad_() for t in (x, r, w))
    h, n = torch.ops.autokernel.fused_res_rmsnorm(xd, rd_, wd, 1e-5)
    torch.autograd.backward([h, n], [up.to(DEV), up.to(DEV)])
    x64, r64, w64 = (t.double().requires_grad_() for t in (x, r, w))
    h64 = (x64 + r64)
    torch.autograd.backward([h64, ops.rmsnorm_ref(h64, w64, 1e-5)], [up.double(), up.double()])
    assert torch.equal(xd.grad, rd_.grad)
    assert torch.allclose(xd.grad.double().cpu(), x64.grad, rtol=tol, atol=tol)
    assert torch.allclose(wd.grad.double().cpu(), w64.grad, rtol=tol, atol=tol * 64)


def test_backward_of_broadcast_upstream_gradient():
    """The gradient of y.sum(0) reaches the backward as an expand-ed tensor
    (stride(0) == 0); the wrapper copies it instead of reading past it."""
    need_gpu()
    g = torch.Generator().manual_seed(14)
    x = torch.randn(32, 512, generator=g)
    w = 1 + 0.1 * torch.randn(512, generator=g)
    up = torch.randn(512, generator=g)
    say("rmsnorm bwd expanded grad")
    xd, wd = x.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
    y = torch.ops.autokernel.rmsnorm(xd, wd, 1e-6)
    y.sum(0).backward(up.to(DEV))
    x64, w64 = x.double().requires_grad_(), w.double().requires_grad_()
    ops.rmsnorm_ref(x64, w64, 1e-6).sum(0).backward(up.double())
    assert torch.allclose(xd.grad.double().cpu(), x64.grad, rtol=1e-4, atol=1e-5)
    assert torch.allclose(wd.grad.double().cpu(), w64.grad, rtol=1e-4, atol=1e-4)
