"""GPU: the no-allocation entry point ak_fused_add_rmsnorm_bwd_noalloc against
ak_fused_add_rmsnorm_bwd (the same kernels with a caller workspace).

Bar: bitwise equal grad_x and grad_weight (both entry points run the same
plan, so the same kernels sum in the same order), on two calls in a row, the
second with a smaller input, so the fixed scratch's leftover contents from
the first call must not leak into the second. Shapes beyond the scratch are
rejected by the argument check before any GPU work.
"""

import pytest
import torch

from gpu_util import gpu, need_gpu, say

pytestmark = gpu
DEV = "cuda"


def _inputs(rows, cols, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(rows, cols, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(cols, generator=g)).to(dtype)
    gh = torch.randn(rows, cols, generator=g).to(dtype)
    gn = torch.randn(rows, cols, generator=g).to(dtype)
    return [t.to(DEV) for t in (h, w, gh, gn)]


def _with_workspace(h, w, gh, gn, eps):
    from kernels.hip import _lib
    gx = torch.empty_like(h)
    gw = torch.empty(h.shape[1], dtype=torch.float32, device=DEV)
    ws = torch.empty(_lib.rmsnorm_bwd_workspace_bytes(*h.shape), dtype=torch.uint8, device=DEV)
    _lib.fused_add_rmsnorm_bwd(h, w, gh, gn, gx, gw, ws, eps)
    return gx, gw


def _no_alloc(h, w, gh, gn, eps):
    from kernels.hip import _lib
    gx = torch.empty_like(h)
    gw = torch.empty(h.shape[1], dtype=torch.float32, device=DEV)
    _lib.fused_add_rmsnorm_bwd_noalloc(h, w, gh, gn, gx, gw, eps)
    return gx, gw


@pytest.mark.parametrize("dtype,first,second,with_dh", [
    (torch.bfloat16, (4096, 4096), (300, 4096), True),    # vector kernel, 1 row per workgroup
    (torch.bfloat16, (20000, 512), (77, 256), False),     # 64-thread rows, 4 slots per workgroup
    (torch.float32, (1000, 16384), (9, 1000), True),      # 16 MiB of partial rows, then generic
    (torch.float16, (513, 4104), (33, 7), True),          # unaligned widths: generic kernel
])
def test_no_alloc_matches_workspace_entry(dtype, first, second, with_dh):
    need_gpu()
    for rows, cols in (first, second):
        say("no-alloc bwd", dtype, rows, cols, with_dh)
        h, w, gh, gn = _inputs(rows, cols, dtype, rows + cols)
        gh = gh if with_dh else None
        ref_x, ref_w = _with_workspace(h, w, gh, gn, 1e-5)
        got_x, got_w = _no_alloc(h, w, gh, gn, 1e-5)
        torch.cuda.synchronize()
        assert torch.equal(got_x, ref_x)
        assert torch.equal(got_w, ref_w)


def test_no_alloc_rejects_shapes_beyond_the_scratch():
    need_gpu()
    from kernels.hip import _lib
    # 256 partial rows x 16392 fp32 columns = 16.8 MB > 16 MiB
    h, w, _, gn = _inputs(512, 16392, torch.float32, 1)
    say("no-alloc too large")
    with pytest.raises(RuntimeError, match="scratch"):
        _no_alloc(h, w, None, gn, 1e-6)
    # without a weight gradient there are no partial rows, so any width runs
    gx = torch.empty_like(h)
    _lib.fused_add_rmsnorm_bwd_noalloc(h, w, None, gn, gx, None, 1e-6)
    ref = torch.empty_like(h)
    _lib.fused_add_rmsnorm_bwd(h, w, None, gn, ref, None, None, 1e-6)
    assert torch.equal(gx, ref)


def test_no_alloc_two_streams_queued_together():
    """Calls queued on two streams without waiting for each other (their
    kernels may run at the same time): each stream owns its own slot of the
    fixed scratch, so both results equal the workspace entry point's bit for
    bit. Repeated with the streams' roles swapped and with a second round of
    calls, so each slot's leftover contents are reused."""
    need_gpu()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    shapes = [(6000, 4096, 11), (3000, 4096, 12)]
    cases = []
    for rows, cols, seed in shapes:
        h, w, gh, gn = _inputs(rows, cols, torch.bfloat16, seed)
        cases.append(((h, w, gh, gn), _with_workspace(h, w, gh, gn, 1e-5)))
    torch.cuda.synchronize()
    for rnd in range(2):
        say("no-alloc two streams, round", rnd)
        outs = []
        order = [0, 1] if rnd == 0 else [1, 0]
        for si, ci in zip(order, [0, 1]):
            with torch.cuda.stream(streams[si]):
                outs.append(_no_alloc(*cases[ci][0], 1e-5))
        torch.cuda.synchronize()
        for (got_x, got_w), (_, (ref_x, ref_w)) in zip(outs, cases):
            assert torch.equal(got_x, ref_x)
            assert torch.equal(got_w, ref_w)
