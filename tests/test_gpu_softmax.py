"""GPU parity: row softmax against the oracle (``reference.py:14-17``).

Bars: fp16 / bf16 outputs within 1 ulp of the fp32-accumulated oracle; fp32
within 1e-5 relative (plus 1e-7 absolute for tiny probabilities); masked
(-inf) entries exactly zero; a row with one finite entry exactly 1.0.
"""

import math

import pytest
import torch

from gpu_util import gpu, max_ulp, need_gpu, say
from oracle import ops

pytestmark = gpu
DEV = "cuda"


def test_c2_causal_softmax_full():
    need_gpu()
    import bench
    from kernels.hip import softmax
    c = bench.gen_c2()
    say("C2 causal softmax fp16 [8, 12, 1024, 1024]")
    xd = c["x"].to(DEV)
    y = softmax.kernel_fn(xd)
    yc = y.cpu()
    ref = ops.softmax_ref(c["x"])
    assert not torch.isnan(yc).any()                                    # every row written
    assert max_ulp(yc, ref) <= 1
    mask = bench.causal_mask(1024)
    assert bool((yc[..., mask] == 0).all())                             # exact zeros
    assert bool((yc[..., 0, 0] == 1.0).all())                           # single finite entry
    nz = (yc != 0).sum(-1)
    assert bool((nz <= torch.arange(1, 1025)).all())
    sums = yc.float().sum(-1)
    assert float((sums - 1).abs().max()) < 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cols", [1, 2, 7, 64, 100, 1000, 1024, 4096, 5000, 8192, 20000, 70000])
def test_softmax_shapes(dtype, cols):
    need_gpu()
    from kernels.hip import softmax
    g = torch.Generator().manual_seed(cols + 1)
    rows = 33 if cols <= 8192 else 4
    x = (4 * torch.randn(rows, cols, generator=g)).to(dtype)
    say("softmax", dtype, rows, cols)
    y = softmax.kernel_fn(x.to(DEV)).cpu()
    ref = ops.softmax_ref(x)
    if dtype == torch.float32:
        d = (y.double() - ref.double()).abs()
        assert bool((d <= 1e-5 * ref.double().abs() + 1e-7).all())
    else:
        assert max_ulp(y, ref) <= 1


def test_softmax_special_values():
    need_gpu()
    from kernels.hip import softmax
    ninf = float("-inf")
    x = torch.tensor([[0.0, ninf, ninf, ninf],
                      [ninf, ninf, ninf, ninf],
                      [1.0, 1.0, 1.0, 1.0],
                      [0.0, math.log(2), math.log(3), ninf]])
    say("softmax special values")
    for dt in (torch.float32, torch.float16):
        y = softmax.kernel_fn(x.to(dt).to(DEV)).float().cpu()
        assert torch.equal(y[0], torch.tensor([1.0, 0, 0, 0]))
        assert bool(torch.isnan(y[1]).all())                              # as F.softmax
        assert torch.allclose(y[2], torch.full((4,), 0.25))
        assert torch.allclose(y[3], torch.tensor([1 / 6, 1 / 3, 1 / 2, 0.0]), atol=1e-3)
        assert y[3, 3] == 0.0
    # wide rows through the generic kernel keep the same special cases
    w = torch.full((2, 70000), ninf)
    w[0, 123] = 5.0
    yw = softmax.kernel_fn(w.to(DEV)).cpu()
    assert yw[0, 123] == 1.0 and float(yw[0].sum()) == 1.0
    assert bool(torch.isnan(yw[1]).all())


def test_softmax_rank_and_determinism():
    need_gpu()
    from kernels.hip import softmax
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 5, 7, 96, generator=g).bfloat16().to(DEV)
    say("softmax rank-4 + determinism")
    ys = [softmax.kernel_fn(x) for _ in range(3)]
    assert ys[0].shape == x.shape
    assert torch.equal(ys[0], ys[1]) and torch.equal(ys[1], ys[2])
    xt = torch.randn(64, 128, generator=g).to(DEV).t()                   # non-contiguous last dim
    yt = softmax.kernel_fn(xt).cpu()
    assert torch.allclose(yt, ops.softmax_ref(xt.cpu()), atol=1e-6)


def test_softmax_grid_stride_and_expanded_rows():
    """Row counts past the 2^20-workgroup grid cap (vector and generic
    kernels) and an expand-ed input (stride(0) == 0)."""
    need_gpu()
    from kernels.hip import softmax
    g = torch.Generator().manual_seed(13)
    for rows, cols in ((4_300_000, 16), (1_100_000, 7)):
        say("softmax grid stride", rows, cols)
        x = 3 * torch.randn(rows, cols, generator=g)
        y = softmax.kernel_fn(x.to(DEV)).cpu()
        ref = ops.softmax_ref(x)
        assert bool(((y - ref).abs() <= 1e-5 * ref.abs() + 1e-7).all())
    xe = torch.randn(1024, generator=g).half().expand(3, 1024)
    say("softmax expanded")
    ye = softmax.kernel_fn(xe.to(DEV)).cpu()
    assert max_ulp(ye, ops.softmax_ref(xe.contiguous())) <= 1
