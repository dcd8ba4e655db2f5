"""GPU parity: RMSNorm and fused residual-add + RMSNorm against the oracle.

Bars (north star): fp32 <= 1e-5 relative; fp16 / bf16 outputs within 1 ulp of
the oracle's fp32-computed, once-rounded value; new_residual bit-exact
(round-to-nearest-even of the exact fp32 sum, which is what the reference's
``x + residual`` produces).
"""

import pytest
import torch

from gpu_util import gpu, max_ulp, need_gpu, rel_err, say
from oracle import ops

pytestmark = gpu

DEV = "cuda"


def _rel_ok_f32(y, ref):
    # elementwise |a-b| <= 1e-5 |b| + 1e-7 * max|b|
    d = (y.double().cpu() - ref.double()).abs()
    bound = 1e-5 * ref.double().abs() + 1e-7 * ref.double().abs().max()
    return bool((d <= bound).all())


def test_c1_rmsnorm_fp32_full():
    need_gpu()
    import bench
    from kernels.hip import rmsnorm
    c = bench.gen_c1()
    say("C1 rmsnorm fp32 [2048, 768]")
    y = rmsnorm.kernel_fn(c["x"].to(DEV), c["w"].to(DEV), c["eps"]).cpu()
    ref = ops.rmsnorm_ref(c["x"], c["w"], c["eps"])
    assert _rel_ok_f32(y, ref), rel_err(y, ref)


def test_c3_fused_bf16_full():
    need_gpu()
    import bench
    from kernels.hip import fused_residual_add_rmsnorm as frn
    c = bench.gen_c3()
    say("C3 fused residual rmsnorm bf16 [16384, 4096]")
    h, y = frn.kernel_fn_dual(c["x"].to(DEV), c["r"].to(DEV), c["w"].to(DEV), eps=c["eps"])
    hr, yr = ops.fused_residual_add_rmsnorm_ref(c["x"], c["r"], c["w"], c["eps"])
    assert torch.equal(h.cpu(), hr)
    assert max_ulp(y, yr) <= 1
    y1 = frn.kernel_fn(c["x"].to(DEV), c["r"].to(DEV), c["w"].to(DEV), eps=c["eps"])
    assert torch.equal(y1.cpu(), y.cpu())


def test_c1_c3_weight_homogeneity_bitwise():
    """Full C1 and C3: y is linear in the weight and doubling it is exact in the
    kernel's fp32 arithmetic and in the final rounding, so y(2w) == 2 y(w)
    bit for bit; new_residual does not depend on the weight."""
    need_gpu()
    import bench
    from kernels.hip import fused_residual_add_rmsnorm as frn
    from kernels.hip import rmsnorm
    c1 = bench.gen_c1()
    x, w = c1["x"].to(DEV), c1["w"].to(DEV)
    assert torch.equal(rmsnorm.kernel_fn(x, 2 * w, c1["eps"]), 2 * rmsnorm.kernel_fn(x, w, c1["eps"]))
    c3 = bench.gen_c3()
    x, r, w = c3["x"].to(DEV), c3["r"].to(DEV), c3["w"].to(DEV)
    h1, y1 = frn.kernel_fn_dual(x, r, w, eps=c3["eps"])
    h2, y2 = frn.kernel_fn_dual(x, r, 2 * w, eps=c3["eps"])
    assert torch.equal(h1, h2) and torch.equal(y2, 2 * y1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cols", [1, 7, 64, 100, 512, 768, 1000, 2048, 4096, 4104, 8192, 16384, 40000, 70000])
def test_rownorm_shapes(dtype, cols):
    need_gpu()
    from kernels.hip import fused_residual_add_rmsnorm as frn
    from kernels.hip import rmsnorm
    g = torch.Generator().manual_seed(cols)
    rows = 37 if cols <= 16384 else 5
    x = (2 * torch.randn(rows, cols, generator=g)).to(dtype)
    r = torch.randn(rows, cols, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(cols, generator=g)).to(dtype)
    say("rownorm", dtype, rows, cols)
    y = rmsnorm.kernel_fn(x.to(DEV), w.to(DEV)).cpu()
    h, yf = frn.kernel_fn_dual(x.to(DEV), r.to(DEV), w.to(DEV))
    hr, yfr = ops.fused_residual_add_rmsnorm_ref(x, r, w)
    yr = ops.rmsnorm_f32_ref(x, w)
    assert torch.equal(h.cpu(), hr)
    if dtype == torch.float32:
        assert _rel_ok_f32(y, yr) and _rel_ok_f32(yf.cpu(), yfr)
    else:
        assert max_ulp(y, yr) <= 1 and max_ulp(yf.cpu(), yfr) <= 1


def test_rownorm_strided_rows_and_edges():
    need_gpu()
    from kernels.hip import fused_residual_add_rmsnorm as frn
    from kernels.hip import rmsnorm
    g = torch.Generator().manual_seed(11)
    big = torch.randn(40, 1040, generator=g).bfloat16()
    x = big[:, :1024]                      # row pitch 1040 elements (16-byte aligned)
    xo = big[:, 3:1027]                    # misaligned start -> scalar path
    w = torch.ones(1024).bfloat16()
    say("rownorm strided")
    for v in (x, xo):
        y = rmsnorm.kernel_fn(v.to(DEV), w.to(DEV)).cpu()
        assert max_ulp(y, ops.rmsnorm_f32_ref(v, w)) <= 1
    z = rmsnorm.kernel_fn(torch.zeros(4, 256, device=DEV), torch.ones(256, device=DEV))
    assert torch.equal(z.cpu(), torch.zeros(4, 256))
    # adversarial magnitudes (the reference harness's near_max transform for fp16)
    xm = (torch.rand(16, 768, generator=g) * 2 - 1).mul(60000).half()
    ym = rmsnorm.kernel_fn(xm.to(DEV), torch.ones(768, dtype=torch.half, device=DEV)).cpu()
    assert torch.isfinite(ym).all() and max_ulp(ym, ops.rmsnorm_f32_ref(xm, torch.ones(768).half())) <= 1
    e = rmsnorm.kernel_fn(torch.empty(0, 64, device=DEV), torch.ones(64, device=DEV))
    assert e.shape == (0, 64)
    h, n = frn.kernel_fn_dual(torch.ones(3, 1, device=DEV), torch.ones(3, 1, device=DEV),
                              torch.full((1,), 2.0, device=DEV), eps=0.0)
    assert torch.equal(h.cpu(), torch.full((3, 1), 2.0)) and torch.equal(n.cpu(), torch.full((3, 1), 2.0))


def test_rownorm_deterministic():
    need_gpu()
    import bench
    from kernels.hip import fused_residual_add_rmsnorm as frn
    c = bench.gen_c3(rows=2048)
    x, r, w = c["x"].to(DEV), c["r"].to(DEV), c["w"].to(DEV)
    say("rownorm determinism")
    outs = [frn.kernel_fn_dual(x, r, w, eps=1e-5)[1] for _ in range(3)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])


def test_rownorm_expanded_views_and_grid_stride():
    """Overlapping rows (an expand-ed residual, stride(0) == 0) are copied by
    the wrapper, not read past the buffer; row counts past the 2^20-workgroup
    grid cap are covered by the grid-stride loops (vector and generic paths)."""
    need_gpu()
    from kernels.hip import fused_residual_add_rmsnorm as frn
    from kernels.hip import rmsnorm
    g = torch.Generator().manual_seed(12)
    x = torch.randn(4, 6, 768, generator=g).bfloat16()
    r1 = torch.randn(768, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(768, generator=g)).bfloat16()
    r = r1.expand(4, 6, 768)
    say("rownorm expanded residual")
    h, y = frn.kernel_fn_dual(x.to(DEV), r1.to(DEV).expand(4, 6, 768), w.to(DEV), eps=1e-5)
    hr, yr = ops.fused_residual_add_rmsnorm_ref(x.reshape(-1, 768), r.reshape(-1, 768), w, 1e-5)
    assert torch.equal(h.cpu().reshape(-1, 768), hr)
    assert max_ulp(y.cpu().reshape(-1, 768), yr) <= 1
    xe = torch.randn(256, generator=g).expand(5, 256)
    ye = rmsnorm.kernel_fn(xe.to(DEV), torch.ones(256, device=DEV)).cpu()
    assert _rel_ok_f32(ye, ops.rmsnorm_f32_ref(xe.contiguous(), torch.ones(256)))
    # 4.3M rows of 16 fp32 (the 64-thread vector kernel, 4 rows per workgroup:
    # > 2^20 workgroups) and 1.1M rows of 7 fp32 (the generic kernel)
    for rows, cols in ((4_300_000, 16), (1_100_000, 7)):
        say("rownorm grid stride", rows, cols)
        xs = torch.randn(rows, cols, generator=g)
        ws = 1 + 0.1 * torch.randn(cols, generator=g)
        ys = rmsnorm.kernel_fn(xs.to(DEV), ws.to(DEV)).cpu()
        assert _rel_ok_f32(ys, ops.rmsnorm_f32_ref(xs, ws))
