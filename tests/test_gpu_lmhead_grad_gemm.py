"""GPU parity: the lm-head gradient GEMMs (ak_lmhead_grad_hidden / _weight).

grad_hidden = dlogits @ W and grad_weight = dlogits^T @ h with fp32
accumulation, checked against fp32 products on the GPU (torch.mm of the
fp32-converted operands). Bar: |out - ref| <= 1e-4 * (|dlogits| @ |W|)
elementwise (fp32 accumulation in a different order), plus half an ulp of
the output type for the 16-bit outputs. Shapes reach every work split:
whole tiles stored directly, K-split tiles summed from partials, both in one
launch, and the M / N / K tails (zero rows past K, zero padding columns of
dlogits, clamped rows past M, masked columns past N).
"""

import pytest
import torch

from gpu_util import gpu, need_gpu, say

pytestmark = gpu
DEV = "cuda"


def _dl(n, vocab, dtype, gen, pad_extra=64):
    """dlogits-like [n, vocab] view of a zero-padded buffer (pitch covers vocab
    rounded up to 64, plus pad_extra)."""
    pitch = -(-vocab // 64) * 64 + pad_extra
    buf = torch.zeros(n, pitch, dtype=dtype)
    buf[:, :vocab] = (1e-3 * torch.randn(n, vocab, generator=gen)).to(dtype)
    buf = buf.to(DEV)
    return buf[:, :vocab]


def _bound(a, b):
    return a.float().abs() @ b.float().abs()


def _check(out, ref, bound, dtype_out, what):
    tol = 1e-4 * bound + 1e-30
    if dtype_out != torch.float32:
        tol = tol + ref.abs() * 2.0 ** -8
    err = (out.float() - ref).abs()
    worst = float((err / tol).max())
    say(f"{what}: max err/tol {worst:.3f}")
    assert worst <= 1.0, what


def _run_pair(n, vocab, d, dtype, gen, mode=0):
    from kernels.hip import _lib
    dl = _dl(n, vocab, dtype, gen)
    W = (0.02 * torch.randn(vocab, d, generator=gen)).to(dtype).to(DEV)
    h = torch.randn(n, d, generator=gen).to(dtype).to(DEV)
    ws_bytes = _lib.lmhead_grad_workspace_bytes(n, vocab, d)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    odt = dtype if mode == _lib.GEMM_OUT_DTYPE else torch.float32
    gh = torch.empty(n, d, dtype=odt, device=DEV)
    gw = torch.empty(vocab, d, dtype=odt, device=DEV)
    _lib.lmhead_grad_hidden(dl, W, gh, mode, ws)
    _lib.lmhead_grad_weight(dl, h, gw, mode, ws)
    torch.cuda.synchronize()
    return dl, W, h, gh, gw


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,vocab,d", [(64, 64, 64), (300, 1000, 64), (1000, 777, 576),
                                       (2048, 8192, 256), (257, 300, 320), (5, 4097, 128),
                                       (512, 66048, 256)])
def test_grad_gemms_match_fp32(dtype, n, vocab, d):
    need_gpu()
    say(f"grad gemms n={n} vocab={vocab} d={d} {dtype}")
    gen = torch.Generator().manual_seed(n + 3 * vocab + 7 * d)
    dl, W, h, gh, gw = _run_pair(n, vocab, d, dtype, gen)
    dlf = dl.float().contiguous()
    _check(gh, torch.mm(dlf, W.float()), _bound(dlf, W), dtype, "grad_hidden")
    dlt = dlf.t().contiguous()
    _check(gw, torch.mm(dlt, h.float()), _bound(dlt, h), dtype, "grad_weight")


@pytest.mark.parametrize("mode", [1, 2])
def test_grad_gemms_fp32_outputs(mode):
    need_gpu()
    from kernels.hip import _lib
    n, vocab, d = 700, 3000, 192
    gen = torch.Generator().manual_seed(11)
    dl = _dl(n, vocab, torch.bfloat16, gen)
    W = (0.02 * torch.randn(vocab, d, generator=gen)).bfloat16().to(DEV)
    h = torch.randn(n, d, generator=gen).bfloat16().to(DEV)
    ws = torch.empty(max(1, _lib.lmhead_grad_workspace_bytes(n, vocab, d)), dtype=torch.uint8, device=DEV)
    base_h = torch.randn(n, d, generator=gen).to(DEV) if mode == 2 else torch.zeros(n, d, device=DEV)
    base_w = torch.randn(vocab, d, generator=gen).to(DEV) if mode == 2 else torch.zeros(vocab, d, device=DEV)
    gh, gw = base_h.clone(), base_w.clone()
    _lib.lmhead_grad_hidden(dl, W, gh, mode, ws)
    _lib.lmhead_grad_weight(dl, h, gw, mode, ws)
    dlf = dl.float().contiguous()
    dlt = dlf.t().contiguous()
    _check(gh - base_h, torch.mm(dlf, W.float()), _bound(dlf, W) + 1e-6 * base_h.abs(), torch.float32,
           "grad_hidden fp32")
    _check(gw - base_w, torch.mm(dlt, h.float()), _bound(dlt, h) + 1e-6 * base_w.abs(), torch.float32,
           "grad_weight fp32")


def test_grad_gemms_c4_shape_and_determinism():
    """The C4 backward's shapes (grad_hidden split 8 ways over 96 tiles,
    grad_weight 512 whole tiles plus 79 split 3 ways), twice: bit-identical."""
    need_gpu()
    from kernels.hip import _lib
    n, vocab, d = 8192, 50304, 768
    gen = torch.Generator().manual_seed(4)
    dl, W, h, gh, gw = _run_pair(n, vocab, d, torch.bfloat16, gen)
    _, _, _, gh2, gw2 = _run_pair(n, vocab, d, torch.bfloat16, torch.Generator().manual_seed(4))
    assert torch.equal(gh, gh2) and torch.equal(gw, gw2)
    dlf = dl.float().contiguous()
    _check(gh, torch.mm(dlf, W.float()), _bound(dlf, W), torch.bfloat16, "c4 grad_hidden")
    dlt = dlf.t().contiguous()
    del dlf
    _check(gw, torch.mm(dlt, h.float()), _bound(dlt, h), torch.bfloat16, "c4 grad_weight")


def test_grad_gemms_c4_homogeneous_bitwise():
    """Both GEMMs are linear in dlogits and doubling it is exact through the
    fp32 accumulation, the K-split partial sums and the final rounding:
    gemm(2 dlogits) == 2 gemm(dlogits) bit for bit at the C4 shape."""
    need_gpu()
    from kernels.hip import _lib
    n, vocab, d = 8192, 50304, 768
    gen = torch.Generator().manual_seed(6)
    dl, W, h, gh, gw = _run_pair(n, vocab, d, torch.bfloat16, gen)
    ws = torch.empty(_lib.lmhead_grad_workspace_bytes(n, vocab, d), dtype=torch.uint8, device=DEV)
    dl2 = (2 * dl).contiguous()
    gh2, gw2 = torch.empty_like(gh), torch.empty_like(gw)
    _lib.lmhead_grad_hidden(dl2, W, gh2, 0, ws)
    _lib.lmhead_grad_weight(dl2, h, gw2, 0, ws)
    assert torch.equal(gh2, 2 * gh) and torch.equal(gw2, 2 * gw)


def test_grad_gemm_workspace_too_small_is_an_error():
    need_gpu()
    from kernels.hip import _lib
    n, vocab, d = 300, 1000, 64
    need = _lib.lmhead_grad_workspace_bytes(n, vocab, d)
    assert need > 0
    gen = torch.Generator().manual_seed(5)
    dl = _dl(n, vocab, torch.bfloat16, gen)
    W = torch.zeros(vocab, d, dtype=torch.bfloat16, device=DEV)
    out = torch.empty(n, d, dtype=torch.bfloat16, device=DEV)
    small = torch.empty(need - 256, dtype=torch.uint8, device=DEV)
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.lmhead_grad_hidden(dl, W, out, 0, small)


def test_grad_hidden_nan_in_k_padding_is_zeroed():
    """The dlogits padding columns [vocab, vocab rounded up to 64) filled with
    NaN: the wrapper zeroes them before the kernel reads its last K block, so
    grad_hidden equals the result from zero padding bit for bit (and is
    finite); a view whose storage ends inside the last row pitch is refused."""
    need_gpu()
    from kernels.hip import _lib
    gen = torch.Generator().manual_seed(41)
    n, vocab, d = 300, 1000, 128
    say("grad_hidden NaN K padding")
    dl0 = _dl(n, vocab, torch.bfloat16, gen)
    pitch = dl0.stride(0)
    buf = torch.full((n, pitch), float("nan"), dtype=torch.bfloat16, device=DEV)
    buf[:, :vocab] = dl0
    W = (0.02 * torch.randn(vocab, d, generator=gen)).bfloat16().to(DEV)
    ws = torch.empty(max(_lib.lmhead_grad_workspace_bytes(n, vocab, d), 1), dtype=torch.uint8, device=DEV)
    want = torch.empty(n, d, dtype=torch.bfloat16, device=DEV)
    got = torch.empty_like(want)
    _lib.lmhead_grad_hidden(dl0, W, want, _lib.GEMM_OUT_DTYPE, ws)
    _lib.lmhead_grad_hidden(buf[:, :vocab], W, got, _lib.GEMM_OUT_DTYPE, ws)
    assert bool(torch.isfinite(got).all()) and torch.equal(got, want)
    short = torch.zeros(n * pitch - 32, dtype=torch.bfloat16, device=DEV)
    view = torch.as_strided(short, (n, vocab), (pitch, 1))
    with pytest.raises(ValueError):
        _lib.lmhead_grad_hidden(view, W, got, _lib.GEMM_OUT_DTYPE, ws)


def test_grad_gemm_wrapper_rejects_mismatched_outputs():
    """Output dtype against out_mode, operand dtype and shapes are checked in
    the wrapper before the C-ABI is called (an fp32 out_mode with a bf16
    output would otherwise store fp32 elements at a bf16 pitch)."""
    need_gpu()
    from kernels.hip import _lib
    gen = torch.Generator().manual_seed(43)
    n, vocab, d = 64, 256, 64
    dl = _dl(n, vocab, torch.bfloat16, gen)
    W = torch.zeros(vocab, d, dtype=torch.bfloat16, device=DEV)
    h = torch.zeros(n, d, dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(max(_lib.lmhead_grad_workspace_bytes(n, vocab, d), 1), dtype=torch.uint8, device=DEV)
    bad = [
        lambda: _lib.lmhead_grad_hidden(dl, W, torch.empty(n, d, dtype=torch.bfloat16, device=DEV),
                                        _lib.GEMM_OUT_F32, ws),
        lambda: _lib.lmhead_grad_hidden(dl, W, torch.empty(n, d, dtype=torch.float32, device=DEV),
                                        _lib.GEMM_OUT_DTYPE, ws),
        lambda: _lib.lmhead_grad_hidden(dl, W.half(), torch.empty(n, d, dtype=torch.bfloat16, device=DEV),
                                        _lib.GEMM_OUT_DTYPE, ws),
        lambda: _lib.lmhead_grad_hidden(dl, W, torch.empty(n + 1, d, dtype=torch.bfloat16, device=DEV),
                                        _lib.GEMM_OUT_DTYPE, ws),
        lambda: _lib.lmhead_grad_weight(dl, h, torch.empty(vocab, d + 64, dtype=torch.bfloat16, device=DEV),
                                        _lib.GEMM_OUT_DTYPE, ws),
        lambda: _lib.lmhead_grad_weight(dl, W, torch.empty(vocab, d, dtype=torch.bfloat16, device=DEV),
                                        _lib.GEMM_OUT_DTYPE, ws),
    ]
    for call in bad:
        with pytest.raises(ValueError):
            call()
