"""Host logic of the drop-in API on the CPU fake backend (CPU tier).

The fake routes every launcher to the oracle, so these tests check what the
Python layer does around the kernels: shapes, dtypes, argument handling,
the ce_fused / chunked CE autograd contracts, the torch.library ops and the
module-swap registry -- the same surfaces the reference's own scripts
exercise (test_ce_features.py, test_chunked_ce.py, test_tier2_parity.py,
test_autokernel_autograd_safety.py).
"""

import math

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import ops


def test_no_cpu_fallback_without_gpu():
    from kernels.hip import rmsnorm, softmax
    x = torch.randn(4, 8)
    with pytest.raises(RuntimeError, match="GPU"):
        rmsnorm.kernel_fn(x, torch.ones(8))
    with pytest.raises(RuntimeError, match="GPU"):
        softmax.kernel_fn(x)


def test_kernel_fns_shapes_and_dtypes(fake_backend):
    from kernels.hip import fused_residual_add_rmsnorm as frn
    from kernels.hip import rmsnorm, softmax
    x = torch.randn(2, 3, 64).bfloat16()
    r = torch.randn(2, 3, 64).bfloat16()
    w = torch.ones(64)
    y = rmsnorm.kernel_fn(x, w)
    assert y.shape == x.shape and y.dtype == x.dtype
    assert torch.equal(y, ops.rmsnorm_f32_ref(x, w.bfloat16()))
    h, n = frn.kernel_fn_dual(x, r, w, eps=1e-5)
    hr, nr_ = ops.fused_residual_add_rmsnorm_ref(x, r, w.bfloat16(), 1e-5)
    assert torch.equal(h, hr) and torch.equal(n, nr_)
    assert torch.equal(frn.kernel_fn(x, r, w, eps=1e-5), nr_)
    s = softmax.kernel_fn(x)
    assert s.shape == x.shape and s.dtype == x.dtype
    with pytest.raises(TypeError):
        rmsnorm.kernel_fn(x.double(), w.double())
    with pytest.raises(ValueError):
        rmsnorm.kernel_fn(x, torch.ones(63))
    with pytest.raises(ValueError):
        frn.kernel_fn(x, r[:, :2], w)


def test_norm_backward_modules(fake_backend):
    """kernels.hip.rmsnorm_backward / fused_residual_rmsnorm_backward: the
    reference's kernel_fn signatures and return contracts (grad_weight fp32;
    the fused form returns grad_x twice)."""
    from kernels.hip import fused_residual_rmsnorm_backward as frb
    from kernels.hip import rmsnorm_backward as rb
    assert rb.KERNEL_TYPE == "rmsnorm_backward" and frb.KERNEL_TYPE == "fused_residual_rmsnorm_backward"
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 3, 64, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(64, generator=g))
    dy = torch.randn(2, 3, 64, generator=g).bfloat16()
    gx, gw = rb.kernel_fn(x, w, dy)
    assert gx.shape == x.shape and gx.dtype == x.dtype and gw.dtype == torch.float32 and gw.shape == (64,)
    ref_x, ref_w = ops.rmsnorm_bwd_ref(x, w.bfloat16(), dy, 1e-6)
    assert torch.equal(gx, ref_x.bfloat16()) and torch.allclose(gw.double(), ref_w, rtol=1e-6)
    gh = torch.randn(2, 3, 64, generator=g).bfloat16()
    a, b, c = frb.kernel_fn(x, w, gh, dy, eps=1e-5)
    assert a is b and c.dtype == torch.float32
    rx, _ = ops.fused_residual_rmsnorm_bwd_ref(x, w.bfloat16(), gh, dy, 1e-5)
    assert torch.equal(a, rx.bfloat16())
    a0, _, _ = frb.kernel_fn(x, w, None, dy)
    assert torch.equal(a0, ops.rmsnorm_bwd_ref(x, w.bfloat16(), dy)[0].bfloat16())
    with pytest.raises(ValueError):
        rb.kernel_fn(x, w, dy[:, :2])
    with pytest.raises(ValueError):
        frb.kernel_fn(x, torch.ones(63), gh, dy)


def test_ce_fused_module_api(fake_backend):
    import kernel
    from kernels import ce_fused
    assert kernel.KERNEL_TYPE == "cross_entropy" and kernel.BACKEND == "hip"
    assert kernel.kernel_fn is ce_fused.kernel_fn
    assert set(ce_fused.TOLERANCES) == {"float16", "bfloat16", "float32"}
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(16, 40, generator=g).half()
    t = torch.randint(0, 40, (16,), generator=g)
    t[2] = -100
    out = ce_fused._get_fwd_module().cross_entropy_fwd_hip(logits, t, 0.0, -100, 0.0, 1, 1, 0.5)
    assert len(out) == 5 and all(o is not None for o in out)
    out = ce_fused._get_fwd_module().cross_entropy_fwd_hip(logits, t, 0.0, -100, 0.0, 0, 0, 1.0)
    assert out[2] is None and out[3] is None and out[4] is None
    loss = ce_fused.kernel_fn(logits, t)
    assert torch.allclose(loss, F.cross_entropy(logits.float(), t), rtol=1e-5)


@pytest.mark.parametrize("mode", ["fused", "tiny"])
@pytest.mark.parametrize("softcap,ls,zw", [(0.0, 0.0, 0.0), (8.0, 0.1, 0.0), (0.0, 0.0, 1e-2),
                                           (8.0, 0.1, 1e-2)])
def test_ce_full_autograd(fake_backend, mode, softcap, ls, zw):
    from kernels.ce_fused import ce_full
    g = torch.Generator().manual_seed(1)
    base = 3 * torch.randn(12, 30, generator=g)
    t = torch.randint(0, 30, (12,), generator=g)
    t[[0, 4]] = -100
    x = base.clone().requires_grad_()
    loss, lse = ce_full(x, t, softcap=softcap, label_smoothing=ls, mode=mode, return_z=True,
                        z_loss_weight=zw)
    (2.0 * loss).backward()
    xr = base.double().requires_grad_()
    xc = softcap * torch.tanh(xr / softcap) if softcap > 0 else xr
    ref = F.cross_entropy(xc, t, ignore_index=-100, label_smoothing=ls)
    if zw > 0:
        valid = (t != -100).double()
        lse_r = torch.logsumexp(xc, -1)
        ref = ref + zw * ((lse_r * valid) ** 2).sum() / valid.sum()
    (2.0 * ref).backward()
    assert torch.allclose(loss.double(), ref.detach(), rtol=1e-5)
    assert torch.allclose(x.grad.double(), xr.grad, atol=1e-6, rtol=1e-4)
    assert torch.allclose(lse.double(), torch.logsumexp(xc.detach(), -1), rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("softcap,ls,zw", [(0.0, 0.0, 0.0), (0.0, 0.0, 1e-3), (10.0, 0.0, 0.0),
                                           (0.0, 0.1, 0.0), (10.0, 0.25, 1e-3)])
def test_chunked_linear_ce(fake_backend, dtype, softcap, ls, zw):
    """Both the fused path (bf16) and the row-chunked path (fp32) against
    F.cross_entropy on materialised fp64 logits, with softcap, label
    smoothing and z-loss."""
    from kernels.hip.chunked_linear_cross_entropy import ChunkedLinearCrossEntropyLoss
    g = torch.Generator().manual_seed(2)
    h0 = torch.randn(2, 20, 64, generator=g)
    W0 = 0.05 * torch.randn(300, 64, generator=g)
    t = torch.randint(0, 300, (2, 20), generator=g)
    t[0, :3] = -100
    h = h0.to(dtype).clone().requires_grad_()
    W = W0.to(dtype).clone().requires_grad_()
    loss = ChunkedLinearCrossEntropyLoss(chunk_size=16, softcap=softcap, label_smoothing=ls,
                                         z_loss_weight=zw)(h, W, t)
    loss.backward()
    hr = h0.to(dtype).double().detach().requires_grad_()
    Wr = W0.to(dtype).double().detach().requires_grad_()
    logits = hr.reshape(-1, 64) @ Wr.t()
    if softcap > 0:
        logits = softcap * torch.tanh(logits / softcap)
    ref = F.cross_entropy(logits, t.reshape(-1), label_smoothing=ls)
    ref.backward()
    if zw > 0:  # z-loss enters the value only (as in the reference module)
        valid = (t.reshape(-1) != -100).double()
        ref = ref + zw * ((torch.logsumexp(logits.detach(), -1) * valid) ** 2).sum() / valid.sum()
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    assert torch.allclose(loss.double(), ref.detach(), rtol=tol)
    assert torch.allclose(h.grad.double(), hr.grad, atol=tol, rtol=tol)
    assert torch.allclose(W.grad.double(), Wr.grad, atol=tol, rtol=tol)


def test_torch_ops_registered_with_fake_and_autograd(fake_backend):
    import kernels.hip._torch_ops  # noqa: F401
    x = torch.randn(6, 32, requires_grad=True)
    w = (1 + 0.1 * torch.randn(32)).requires_grad_()
    y = torch.ops.autokernel.rmsnorm(x, w)
    y.sum().backward()
    xr = x.detach().double().requires_grad_()
    wr = w.detach().double().requires_grad_()
    (xr / torch.sqrt(xr.pow(2).mean(-1, keepdim=True) + 1e-6) * wr).sum().backward()
    assert torch.allclose(x.grad.double(), xr.grad, atol=1e-5)
    assert torch.allclose(w.grad.double(), wr.grad, atol=1e-5)
    r = torch.randn(6, 32, requires_grad=True)
    x.grad = None
    h, n = torch.ops.autokernel.fused_res_rmsnorm(x, r, w, 1e-5)
    (h.sum() + (n * n).sum()).backward()
    assert x.grad is not None and torch.equal(x.grad, r.grad)
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        fx = torch.empty(3, 16)
        out = torch.ops.autokernel.fused_res_rmsnorm(fx, fx, torch.empty(16))
        assert out[0].shape == (3, 16)
    dA = torch.rand(2, 7, 3, requires_grad=True)
    dBx = torch.randn(2, 7, 3, requires_grad=True)
    C = torch.randn(2, 7, 3, requires_grad=True)
    D = torch.randn(3, requires_grad=True)
    xx = torch.randn(2, 7, 3, requires_grad=True)
    torch.ops.autokernel.selective_scan(dA, dBx, C, D, xx).pow(2).sum().backward()
    ins = [t.detach().double().requires_grad_() for t in (dA, dBx, C, D, xx)]
    ops.diag_scan_ref(*ins).double().pow(2).sum().backward()
    ref = [t for t in (dA, dBx, C, D, xx)]
    # the oracle computes in fp32; compare against its autograd
    ins32 = [t.detach().float().requires_grad_() for t in ref]
    ops.diag_scan_ref(*ins32).pow(2).sum().backward()
    for a, b in zip(ref, ins32):
        assert torch.allclose(a.grad, b.grad, rtol=1e-4, atol=1e-4)


def test_selective_scan_fn_api(fake_backend):
    from kernels.hip.selective_scan import selective_scan_fn
    g = torch.Generator().manual_seed(3)
    u = torch.randn(2, 4, 20, generator=g)
    delta = 0.5 * torch.rand(2, 4, 20, generator=g)
    A = -torch.rand(4, 8, generator=g)
    B = torch.randn(2, 8, 20, generator=g)
    C = torch.randn(2, 8, 20, generator=g)
    out, last = selective_scan_fn(u, delta, A, B, C, torch.ones(4), return_last_state=True)
    ref, rl = ops.selective_scan_ref(u, delta, A, B, C, torch.ones(4), return_last_state=True)
    assert torch.allclose(out, ref) and torch.allclose(last, rl)
    # input-independent B / C ([dim, dstate]) and complex A
    B2, C2 = torch.randn(4, 8, generator=g), torch.randn(4, 8, generator=g)
    for bb, cc in ((B2, C), (B, C2), (B2, C2)):
        out2 = selective_scan_fn(u, delta, A, bb, cc, torch.ones(4))
        assert torch.allclose(out2, ops.selective_scan_ref(u, delta, A, bb, cc, torch.ones(4)))
    # complex A: B / C real [b, n, 2l] of (re, im) pairs or complex [dim, n]
    Ac = torch.complex(A, torch.rand(4, 8, generator=g) * 3.0)
    with pytest.raises(ValueError, match="2 \\* seqlen"):
        selective_scan_fn(u, delta, Ac, B, C)
    with pytest.raises(ValueError, match="real"):
        selective_scan_fn(u, delta, Ac, torch.complex(B, B), C)
    Bx, Cx = torch.randn(2, 8, 40, generator=g), torch.randn(2, 8, 40, generator=g)
    Cc = torch.complex(C2, torch.randn(4, 8, generator=g))
    outc, lastc = selective_scan_fn(u, delta, Ac, Bx, Cc, torch.ones(4), return_last_state=True)
    refc, rlc = ops.selective_scan_complex_ref(u, delta, Ac, Bx, Cc, torch.ones(4), return_last_state=True)
    assert torch.allclose(outc, refc.float(), atol=1e-5) and lastc.dtype == torch.complex64
    assert torch.allclose(lastc, rlc.to(torch.complex64), atol=1e-5)
    lc = [t.clone().requires_grad_() for t in (Ac, Bx, Cc)]
    selective_scan_fn(u, delta, lc[0], lc[1], lc[2], torch.ones(4)).sum().backward()
    assert lc[0].grad.dtype == torch.complex64 and lc[0].grad.shape == (4, 8)
    assert lc[1].grad.dtype == torch.float32 and lc[1].grad.shape == (2, 8, 40)
    assert lc[2].grad.dtype == torch.complex64 and lc[2].grad.shape == (4, 8)
    gref = ops.selective_scan_complex_bwd_ref(u, delta, Ac, Bx, Cc, torch.ones_like(u), torch.ones(4))
    assert torch.allclose(lc[0].grad, gref[2].to(torch.complex64), rtol=1e-4, atol=1e-5)
    assert torch.allclose(lc[1].grad, gref[3].float(), rtol=1e-4, atol=1e-5)
    with pytest.raises(ValueError):
        selective_scan_fn(u, delta, A, torch.randn(5, 8), C)
    Bl = B2.clone().requires_grad_()
    selective_scan_fn(u, delta, A, Bl, C).sum().backward()
    assert Bl.grad.shape == (4, 8) and Bl.grad.dtype == torch.float32
    # backward: the autograd function hands the layouts it normalised to the
    # backward entry point and maps the gradients back (dB / dC squeezed to
    # B's / C's [b, n, l], dtype casts by autograd)
    D, z, bias = torch.randn(4, generator=g), torch.randn(2, 4, 20, generator=g), torch.rand(4, generator=g)
    dout = torch.randn(2, 4, 20, generator=g)
    leaves = [t.clone().requires_grad_() for t in (u, delta, A, B, C, D, z, bias)]
    selective_scan_fn(*leaves[:5], D=leaves[5], z=leaves[6], delta_bias=leaves[7],
                      delta_softplus=True).backward(dout)
    ref = ops.selective_scan_bwd_ref(u, delta, A, B, C, dout, D, z, bias, True)
    order = (0, 1, 2, 3, 4, 5, 6, 7)  # du ddelta dA dB dC dD dz dbias
    for leaf, i in zip(leaves, order):
        assert leaf.grad.shape == leaf.shape
        assert torch.allclose(leaf.grad.double(), ref[i], rtol=1e-5, atol=1e-6)
    uu = u.clone().requires_grad_()
    selective_scan_fn(uu, delta, A, B, C).backward(dout)
    assert torch.allclose(uu.grad.double(), ops.selective_scan_bwd_ref(u, delta, A, B, C, dout)[0],
                          rtol=1e-5, atol=1e-6)


def test_selective_scan_cuda_binding_api(fake_backend):
    """kernels.hip.selective_scan_cuda mirrors the reference binding's fwd /
    bwd argument order and return lists (selective_scan.cpp:227-335, :339-490)."""
    from kernels.hip import selective_scan_cuda
    g = torch.Generator().manual_seed(5)
    u = torch.randn(2, 4, 20, generator=g)
    delta = 0.5 * torch.rand(2, 4, 20, generator=g)
    A = -torch.rand(4, 8, generator=g)
    B = torch.randn(2, 8, 20, generator=g)
    C = torch.randn(2, 8, 20, generator=g)
    D, z, bias = torch.randn(4, generator=g), torch.randn(2, 4, 20, generator=g), torch.rand(4, generator=g)
    out, x, out_z = selective_scan_cuda.fwd(u, delta, A, B, C, D, z, bias, True)
    assert x.shape == (2, 4, 1, 16) and x.dtype == torch.float32
    assert torch.allclose(out, ops.selective_scan_ref(u, delta, A, B, C, D, None, bias, True))
    assert torch.allclose(out_z, ops.selective_scan_ref(u, delta, A, B, C, D, z, bias, True))
    xs = ops.selective_scan_chunk_states_ref(u, delta, A, B, bias, True)
    assert torch.allclose(x.double(), xs.reshape(2, 4, 1, 16), rtol=1e-5, atol=1e-6)
    out2, x2 = selective_scan_cuda.fwd(u, delta, A, B, C, None, None, None, False)
    assert x2.shape == (2, 4, 1, 16)
    dout = torch.randn(2, 4, 20, generator=g)
    dz_buf = torch.empty(2, 4, 20)
    res = selective_scan_cuda.bwd(u, delta, A, B, C, D, z, bias, dout, x, out, dz_buf, True, True)
    assert len(res) == 9
    ref = ops.selective_scan_bwd_ref(u, delta, A, B, C, dout, D, z, bias, True)
    for got, want in zip(res[:5], ref[:5]):
        assert got.shape == want.shape and torch.allclose(got.double(), want, rtol=1e-5, atol=1e-6)
    assert torch.allclose(res[5].double(), ref[5], rtol=1e-5, atol=1e-6)   # dD
    assert torch.allclose(res[6].double(), ref[7], rtol=1e-5, atol=1e-6)   # ddelta_bias
    assert res[7] is dz_buf and torch.allclose(res[7].double(), ref[6], rtol=1e-5, atol=1e-6)
    assert torch.allclose(res[8], out_z)
    res = selective_scan_cuda.bwd(u, delta, A, B, C, None, None, None, dout, x2, out2, None, False, False)
    assert len(res) == 7 and res[5] is None and res[6] is None
    # complex weights: x complex64 [batch, dim, n_chunks, 2 * dstate]; dA complex,
    # a variable dB real [batch, dstate, 2 seqlen], a constant dC complex
    Ac = torch.complex(A, torch.rand(4, 8, generator=g))
    Bx = torch.randn(2, 8, 40, generator=g)
    Cc = torch.complex(torch.randn(4, 8, generator=g), torch.randn(4, 8, generator=g))
    outc, xc, outc_z = selective_scan_cuda.fwd(u, delta, Ac, Bx, Cc, D, z, bias, True)
    assert xc.shape == (2, 4, 1, 16) and xc.dtype == torch.complex64
    xsc = ops.selective_scan_complex_chunk_states_ref(u, delta, Ac, Bx, bias, True)
    assert torch.allclose(xc, xsc.reshape(2, 4, 1, 16).to(torch.complex64), rtol=1e-5, atol=1e-6)
    assert torch.allclose(outc, ops.selective_scan_complex_ref(u, delta, Ac, Bx, Cc, D, None, bias, True).float(),
                          rtol=1e-5, atol=1e-5)
    res = selective_scan_cuda.bwd(u, delta, Ac, Bx, Cc, D, z, bias, dout, xc, outc, None, True, False)
    refc = ops.selective_scan_complex_bwd_ref(u, delta, Ac, Bx, Cc, dout, D, z, bias, True)
    assert res[2].dtype == torch.complex64 and res[3].dtype == torch.float32 and res[4].dtype == torch.complex64
    for got, want in zip(res[:5], refc[:5]):
        assert got.shape == want.shape
        assert torch.allclose(got.to(want.dtype), want, rtol=1e-4, atol=1e-5)


# ---------------------------------------------------------------------------
# Registry
# ---------------------------------------------------------------------------

class RMSNorm(nn.Module):
    def __init__(self, d, eps=1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.eps = eps

    def forward(self, x):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps) * self.weight


class Attn(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.proj = nn.Linear(d, d, bias=False)

    def forward(self, x, freqs_cis):
        return self.proj(x)


class Block(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.attention = Attn(d)
        self.attention_norm = RMSNorm(d)
        self.feed_forward = nn.Sequential(nn.Linear(d, 2 * d), nn.SiLU(), nn.Linear(2 * d, d))
        self.ffn_norm = RMSNorm(d)

    def forward(self, x, freqs_cis):
        h = x + self.attention(self.attention_norm(x), freqs_cis)
        return h + self.feed_forward(self.ffn_norm(h))


class Tiny(nn.Module):
    def __init__(self, d=32, n=2):
        super().__init__()
        self.layers = nn.ModuleList([Block(d) for _ in range(n)])
        self.norm = RMSNorm(d)

    def forward(self, x):
        for b in self.layers:
            x = b(x, None)
        return self.norm(x)


def test_registry_patterns_and_priorities():
    import autokernel
    from autokernel._patterns import ALL_PATTERNS
    assert autokernel.list_patterns() == ["fused_residual_rmsnorm", "fused_griffin_block", "fused_qkv",
                                          "rmsnorm", "fused_silu_gate_mul", "silu_gate_mul",
                                          "rotary_embedding"]
    prio = {p.name: p.priority for p in ALL_PATTERNS}
    assert prio == {"fused_residual_rmsnorm": 100, "fused_griffin_block": 95, "fused_qkv": 90,
                    "rmsnorm": 50, "fused_silu_gate_mul": 45, "silu_gate_mul": 40,
                    "rotary_embedding": 30}


def test_optimize_report_restore(fake_backend):
    import autokernel
    torch.manual_seed(0)
    model = Tiny()
    x = torch.randn(2, 5, 32)
    ref = model(x)
    orig_keys = set(model.state_dict())
    model = autokernel.optimize(model, training=True)
    rep = autokernel.report(model)
    assert rep["status"] == "optimized"
    assert rep["patterns"]["fused_residual_rmsnorm"]["modules_replaced"] == 2
    assert rep["patterns"]["rmsnorm"]["modules_replaced"] >= 1
    keys = set(model.state_dict())
    assert "layers.0.ffn_norm_weight" in keys and "layers.0.ffn_norm.weight" not in keys
    out = model(x)
    assert torch.allclose(out, ref, atol=1e-5)
    out.pow(2).mean().backward()
    for name, p in model.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), name
    autokernel.restore(model)
    assert set(model.state_dict()) == orig_keys
    assert autokernel.report(model)["status"] == "not optimized"


def test_optimize_include_exclude(fake_backend):
    import autokernel
    m = autokernel.optimize(Tiny(), training=True, include=["rmsnorm"])
    assert list(autokernel.report(m)["patterns"]) == ["rmsnorm"]
    m = autokernel.optimize(Tiny(), training=True, exclude=["rmsnorm", "fused_residual_rmsnorm"])
    assert autokernel.report(m)["patterns"] == {}


def test_replacements_route_through_custom_ops(fake_backend):
    """Static audit of the module swaps (as the reference's
    scripts/audit_autokernel_replacements.py does with ast): every call in a
    replacement's forward goes through a registered torch.ops.autokernel op
    (autograd-safe) or ordinary module / tensor methods, never through a raw
    kernel entry (kernel_fn / kernel_fn_dual / the ctypes library), which
    would sever autograd. The op attributes are checked to be those ops."""
    import ast
    import inspect

    import autokernel
    from autokernel import _patterns

    tree = ast.parse(inspect.getsource(_patterns))
    classes = [n for n in tree.body if isinstance(n, ast.ClassDef) and n.name.endswith("Replacement")]
    assert len(classes) == 2
    unsafe = ("self.kernel_fn", "self.kernel_fn_dual", "_lib.", "_get_fwd_module", "_get_bwd_module")
    for cls in classes:
        fwd = next(f for f in cls.body if isinstance(f, ast.FunctionDef) and f.name == "forward")
        calls = [ast.unparse(c.func) for c in ast.walk(fwd) if isinstance(c, ast.Call)]
        assert not [c for c in calls if any(c.startswith(u) or u in c for u in unsafe)], (cls.name, calls)
        assert any(c.startswith("self._autograd_") for c in calls), (cls.name, calls)
    model = autokernel.optimize(Tiny(), training=True)
    ops_seen = set()
    for m in model.modules():
        for attr in ("_autograd_op", "_autograd_dual"):
            op = getattr(m, attr, None)
            if op is not None:
                assert isinstance(op, torch._ops.OpOverloadPacket), (type(m).__name__, attr)
                ops_seen.add(str(op))
    assert ops_seen == {"autokernel.rmsnorm", "autokernel.fused_res_rmsnorm"}, ops_seen


def test_selective_scan_fn_keeps_states_only_when_recording(fake_backend, monkeypatch):
    """The forward keeps its 16-step states for the backward only when autograd
    records the call: not under torch.no_grad() (inference with parameters
    that require grad), nor with AUTOKERNEL_SCAN_RECOMPUTE's switch off."""
    from kernels.hip import _lib
    from kernels.hip import selective_scan as ss
    seen = []
    fake_scan = _lib.selective_scan

    def spy(*args, **kw):
        seen.append(kw.get("checkpoints") is not None)
        return fake_scan(*args, **kw)

    monkeypatch.setattr(_lib, "selective_scan", spy)
    g = torch.Generator().manual_seed(4)
    u = torch.randn(1, 4, 32, generator=g)
    delta = torch.rand(1, 4, 32, generator=g) * 0.5
    A = torch.nn.Parameter(-torch.rand(4, 8, generator=g) - 0.5)
    B = torch.randn(1, 8, 32, generator=g)
    C = torch.randn(1, 8, 32, generator=g)
    z = torch.randn(1, 4, 32, generator=g)
    with torch.no_grad():
        ss.selective_scan_fn(u, delta, A, B, C, z=z)
    out = ss.selective_scan_fn(u, delta, A, B, C, z=z)
    out.sum().backward()
    assert A.grad is not None and torch.isfinite(A.grad).all()
    monkeypatch.setattr(ss, "SAVE_STATES", False)
    ss.selective_scan_fn(u, delta, A, B, C, z=z).sum().backward()
    assert seen == [False, True, False]


def test_rows_view_rejects_overlapping_rows_and_as_rows_copies():
    from kernels.hip import _lib
    e = torch.randn(768).expand(4, 768)
    # the pitch is passed on unchanged (0), so the C-ABI's pitch check rejects it
    assert _lib._rows_view(e, "x") == 0
    assert _lib._rows_view(torch.randn(1, 768).expand(1, 768), "x") == 768
    c = _lib.as_rows(e, 768)
    assert c.stride() == (768, 1) and torch.equal(c, e)
    big = torch.randn(6, 800)
    v = _lib.as_rows(big[:, :768], 768)        # pitch 800 >= cols: no copy
    assert v.data_ptr() == big.data_ptr() and v.stride() == (800, 1)
    t = _lib.as_rows(torch.randn(768, 6).t(), 768)
    assert t.is_contiguous()


def test_rmsnorm_replacement_takes_the_modules_own_eps(fake_backend):
    """HF-style norms keep eps in ``variance_epsilon``; the swap must use it
    (and GemmaRMSNorm's 1 + weight scaling)."""
    import torch.nn as nn
    from autokernel._patterns import _RMSNormReplacement, _norm_eps
    from kernels.hip.rmsnorm import kernel_fn

    class LlamaRMSNorm(nn.Module):
        def __init__(self, d, eps):
            super().__init__()
            self.weight = nn.Parameter(1 + 0.1 * torch.randn(d))
            self.variance_epsilon = eps

        def forward(self, x):
            v = x.float().pow(2).mean(-1, keepdim=True)
            return self.weight * (x.float() * torch.rsqrt(v + self.variance_epsilon))

    class GemmaRMSNorm(LlamaRMSNorm):
        def forward(self, x):
            v = x.float().pow(2).mean(-1, keepdim=True)
            return (1 + self.weight) * (x.float() * torch.rsqrt(v + self.variance_epsilon))

    x = 0.01 * torch.randn(3, 5, 32)   # small rows: eps matters
    for cls in (LlamaRMSNorm, GemmaRMSNorm):
        m = cls(32, 1e-2)
        rep = _RMSNormReplacement(m, kernel_fn)
        assert rep.eps == 1e-2
        assert torch.allclose(rep(x), m(x), rtol=1e-5, atol=1e-6)
    assert _norm_eps(nn.Module()) == 1e-6
    assert _norm_eps(nn.RMSNorm(8, eps=3e-5)) == 3e-5
    assert _norm_eps(nn.RMSNorm(8)) == torch.finfo(torch.float32).eps


def test_harness_configs_and_compare():
    """The harness's KERNEL_CONFIGS cover the kernel set with the reference's
    entry fields; its comparison treats matching NaN / Inf as equal and
    reports the first mismatch."""
    import harness
    for k in ("softmax", "cross_entropy", "rmsnorm", "fused_residual_add_rmsnorm", "selective_scan"):
        spec = harness.KERNEL_CONFIGS[k]
        assert spec.kernel_type == k and spec.test_sizes and spec.edge_sizes and spec.test_dtypes
        assert all(dt in spec.tolerances for dt in spec.test_dtypes)
        lbl, size = spec.test_sizes[0]
        assert spec.flops_fn(size) > 0 and spec.bytes_fn(size, spec.test_dtypes[0]) > 0
    assert "matmul" not in harness.KERNEL_CONFIGS
    a = torch.tensor([1.0, float("nan"), float("inf"), 2.0])
    b = torch.tensor([1.0 + 1e-7, float("nan"), float("inf"), 2.0])
    assert harness.compare(a, b, 1e-6, 0.0)["match"]
    c = harness.compare(a, torch.tensor([1.0, float("nan"), float("inf"), 2.1]), 1e-3, 1e-3)
    assert not c["match"] and "max_abs_error" in c["reason"]
    assert not harness.compare(a, a[:3], 1.0, 1.0)["match"]
    # the eager references follow reference.py with fp32 arithmetic
    x = torch.randn(4, 33).half()
    assert torch.allclose(harness._softmax_ref({"x": x}).float(), torch.softmax(x.float(), -1), atol=1e-3)
    w = torch.randn(33).half()
    r = harness._fused_ref({"x": x, "residual": x, "weight": w})
    assert torch.equal(r, ops.fused_residual_add_rmsnorm_ref(x, x, w, 1e-6)[1])


def test_harness_stages_run_on_the_fake_backend(fake_backend, monkeypatch):
    """The five correctness stages and their verdicts, driven on the CPU
    through the oracle-backed launchers (device 'cpu'); a planted error in the
    kernel makes the sweep fail."""
    import harness
    from kernels.hip import rmsnorm
    spec = harness.KernelSpec(
        "rmsnorm", [("tiny", {"M": 8, "N": 64}), ("small", {"M": 16, "N": 96})], [torch.float32],
        {torch.float32: {"atol": 1e-5, "rtol": 1e-5}}, harness._rms_inputs, harness._rms_ref,
        rmsnorm.kernel_fn, lambda s: 6 * s["M"] * s["N"], lambda s, dt: 8 * s["M"] * s["N"],
        [("edge_7", {"M": 7, "N": 7})])
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a: None)
    res = harness.run_correctness(spec, device="cpu", log=lambda *a: None)
    assert res["correctness"] == "PASS", res
    assert all(res[k].startswith("PASS") for k in ("smoke_test", "shape_sweep", "numerical_stability",
                                                   "determinism", "edge_cases"))
    bad = harness.KernelSpec(**{**spec.__dict__, "kernel_fn": lambda x, weight: rmsnorm.kernel_fn(x, weight) * 1.01})
    res = harness.run_correctness(bad, device="cpu", log=lambda *a: None)
    assert res["correctness"] == "FAIL" and res["smoke_test"] == "FAIL"


def test_optimized_model_context_swaps_and_restores(fake_backend):
    """verify.OptimizedModelContext: RMSNorm modules and pre-norm blocks are
    replaced inside the context (outputs within tolerance of the original
    model) and every original module object is back afterwards, in either
    replacement order."""
    import torch.nn as nn
    import verify

    class Norm(nn.Module):
        def __init__(self, d):
            super().__init__()
            self.weight = nn.Parameter(1 + 0.1 * torch.randn(d))
            self.eps = 1e-5

        def forward(self, x):
            return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps) * self.weight

    class Block(nn.Module):
        def __init__(self, d):
            super().__init__()
            self.attention = lambda x, f: x * 0.5  # stand-in mixer
            self.attention_norm = Norm(d)
            self.feed_forward = nn.Linear(d, d)
            self.ffn_norm = Norm(d)

        def forward(self, x, freqs_cis):
            h = x + self.attention(self.attention_norm(x), freqs_cis)
            return h + self.feed_forward(self.ffn_norm(h))

    class Model(nn.Module):
        def __init__(self, d=32):
            super().__init__()
            self.layers = nn.ModuleList([Block(d), Block(d)])
            self.norm = Norm(d)

        def forward(self, x):
            for l in self.layers:
                x = l(x, None)
            return self.norm(x)

    torch.manual_seed(0)
    m = Model()
    x = torch.randn(2, 5, 32)
    before = {n: mod for n, mod in m.named_modules()}
    ref = m(x)
    for order in ((0, 1), (1, 0)):
        reps = [verify.KernelReplacement("fused_residual_add_rmsnorm", rank=order[0]),
                verify.KernelReplacement("rmsnorm", rank=order[1]),
                verify.KernelReplacement("rotary_embedding", rank=2)]
        ctx = verify.OptimizedModelContext(m, reps)
        with ctx as mm:
            out = mm(x)
            kinds = {type(mod).__name__ for mod in mm.modules()}
            assert "_FusedResidualRMSNormBlockReplacement" in kinds and "_RMSNormReplacement" in kinds
        assert any("rotary_embedding" in n for n in ctx.notes)
        assert torch.allclose(out, ref, rtol=1e-4, atol=1e-5)
        after = {n: mod for n, mod in m.named_modules()}
        assert after.keys() == before.keys() and all(after[k] is before[k] for k in before)
    res = verify.verify_model.__doc__
    assert res
    cmp = verify.compare_outputs(ref, ref + 1e-6, torch.float32)
    assert cmp["correctness"] == "PASS"
    bad = verify.compare_outputs(ref, ref.clone().fill_(float("nan")), torch.float32)
    assert bad["correctness"] == "FAIL" and "NaN" in bad["reason"]


def test_lmhead_backward_vocab_range_plan(monkeypatch):
    """The lm-head backward's vocab ranges under a dlogits budget: they tile
    the vocabulary in order, every range but the last is whole 256-column
    tiles, none exceeds the budget's width (one tile at least), and their
    number is the fewest that fit. At the C4 shape the plans are the measured
    ones: even shares rounded to whole rounds of the tile kernel's 256
    persistent workgroups (8 vocab tiles x 32 token tiles)."""
    import random
    from kernels.hip import chunked_linear_cross_entropy as clce
    c4 = {512: [96, 96 + 100.5], 256: [48, 96, 144, 196.5], 128: [32, 64, 96, 128, 160, 192, 196.5],
          4096: [196.5]}
    for mb, ends in c4.items():
        monkeypatch.setattr(clce, "GRAD_LOGITS_BUDGET", mb << 20)
        assert [v1 / 256 for _, v1 in clce._vocab_ranges(8192, 50304, 2, 256)] == ends
    rng = random.Random(0)
    for _ in range(3000):
        n, vocab = rng.randint(1, 20000), rng.randint(1, 300000)
        elem, cus = rng.choice([2, 4]), rng.choice([256, 304, 80, 1])
        monkeypatch.setattr(clce, "GRAD_LOGITS_BUDGET", rng.randint(1, 1 << 32))
        r = clce._vocab_ranges(n, vocab, elem, cus)
        tiles = -(-vocab // 256)
        cap = max(1, min(tiles, clce.GRAD_LOGITS_BUDGET // (n * elem * 256)))
        assert r[0][0] == 0 and r[-1][1] == vocab
        assert all(a[1] == b[0] for a, b in zip(r, r[1:])) and all(v1 > v0 for v0, v1 in r)
        assert all((v1 - v0) % 256 == 0 for v0, v1 in r[:-1])
        assert max(-(-(v1 - v0) // 256) for v0, v1 in r) <= cap
        assert len(r) == -(-tiles // cap)
