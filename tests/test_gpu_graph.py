"""HIP graph capture of the kernel entry points.

The C ABI allocates nothing and records no memset, so a caller can capture
its calls in a HIP graph (torch.cuda.CUDAGraph). Each family's forward and
backward entry points are captured once, then replayed several times with
eager work (the outputs overwritten) and synchronisations between the
replays. Every replay must reproduce the eager results bit for bit.
Workspaces the Python launchers allocate inside the capture come from the
graph's private memory pool.
"""

import torch
import torch.nn.functional as F

from gpu_util import gpu, need_gpu, say

pytestmark = gpu
DEV = "cuda"


def test_capture_and_replay_all_families():
    need_gpu()
    from kernels.hip import _lib
    g = torch.Generator().manual_seed(3)
    d = lambda t: t.to(DEV)
    # norms
    x = d(torch.randn(256, 1024, generator=g).bfloat16())
    r = d(torch.randn(256, 1024, generator=g).bfloat16())
    w = d((1 + 0.02 * torch.randn(1024, generator=g)).bfloat16())
    gy = d(torch.randn(256, 1024, generator=g).bfloat16())
    y1, h2, y2, gx = (torch.empty_like(x) for _ in range(4))
    gw = torch.empty(1024, device=DEV)
    ws_n = torch.empty(_lib.rmsnorm_bwd_workspace_bytes(256, 1024), dtype=torch.uint8, device=DEV)
    # softmax and CE over logits
    xs = d((3 * torch.randn(64, 1000, generator=g)).half())
    ys = torch.empty_like(xs)
    logits = d(torch.randn(64, 5000, generator=g).bfloat16())
    t = d(torch.randint(0, 5000, (64,), generator=g))
    losses = torch.empty(64, device=DEV)
    lse = torch.empty(64, device=DEV)
    # lm-head + CE
    hid = d(torch.randn(512, 256, generator=g).bfloat16())
    W = d((0.05 * torch.randn(3000, 256, generator=g)).bfloat16())
    tt = d(torch.randint(0, 3000, (512,), generator=g))
    loss = torch.empty((), device=DEV)
    lse2 = torch.empty(512, device=DEV)
    nv = torch.empty(1, dtype=torch.int64, device=DEV)
    ws_l = torch.empty(_lib.lmhead_ce_workspace_bytes(512, 3000), dtype=torch.uint8, device=DEV)
    one = torch.ones(1, device=DEV)
    den = torch.full((1,), 512.0, device=DEV)
    # dlogits in a buffer whose zeroed padding covers vocab rounded up to 64
    # (what the gradient GEMMs read)
    dz_l = torch.zeros(512, 3008 + 64, dtype=torch.bfloat16, device=DEV)[:, :3000]
    g_h = torch.empty(512, 256, dtype=torch.bfloat16, device=DEV)
    g_w = torch.empty(3000, 256, dtype=torch.bfloat16, device=DEV)
    ws_g = torch.empty(_lib.lmhead_grad_workspace_bytes(512, 3000, 256), dtype=torch.uint8, device=DEV)
    # Mamba-1 scan
    u = d(torch.randn(2, 32, 256, generator=g).bfloat16())
    delta = d(F.softplus(0.5 * torch.randn(2, 32, 256, generator=g) - 2))
    A = d(-torch.rand(32, 16, generator=g) - 0.5)
    B = d(torch.randn(2, 1, 16, 256, generator=g).bfloat16())
    C = d(torch.randn(2, 1, 16, 256, generator=g).bfloat16())
    Dv = d(torch.ones(32))
    z = d(torch.randn(2, 32, 256, generator=g).bfloat16())
    dout = d(torch.randn(2, 32, 256, generator=g).bfloat16())
    out = torch.empty_like(u)
    du, dzs = torch.empty_like(u), torch.empty_like(u)
    ddelta = torch.empty_like(delta)
    dA, dD = torch.empty_like(A), torch.empty_like(Dv)
    dB, dC = torch.empty_like(B), torch.empty_like(C)

    def run():
        _lib.rmsnorm(x, w, y1, 1e-6)
        _lib.fused_add_rmsnorm(x, r, w, h2, y2, 1e-5)
        _lib.rmsnorm_bwd(h2, w, gy, gx, gw, ws_n, 1e-5)
        _lib.softmax(xs, ys)
        _lib.ce_fwd(logits, t, losses, lse, None, None, None, 30.0, -100, 0.1, 1.0)
        _lib.lmhead_ce(hid, W, tt, loss, lse2, None, nv, ws_l, -100, 0.0, 0.0)
        _lib.lmhead_ce_bwd(hid, W, tt, lse2, one, den, dz_l, -100)
        _lib.lmhead_grad_hidden(dz_l, W, g_h, _lib.GEMM_OUT_DTYPE, ws_g)
        _lib.lmhead_grad_weight(dz_l, hid, g_w, _lib.GEMM_OUT_DTYPE, ws_g)
        _lib.selective_scan(u, delta, A, B, C, Dv, z, None, out, None, False)
        _lib.selective_scan_bwd(u, delta, A, B, C, Dv, z, None, dout, du, ddelta, dA, dB, dC, dD,
                                dzs, None, False)

    outs = [y1, h2, y2, gx, gw, ys, losses, lse, loss, lse2, nv, dz_l, g_h, g_w, out, du, ddelta, dA,
            dB, dC, dD, dzs]
    say("graph: eager reference")
    run()
    torch.cuda.synchronize()
    ref = [o.clone() for o in outs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    say("graph: capture")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    torch.cuda.synchronize()
    for i in range(4):
        for o in outs:
            o.fill_(-1 if o.dtype == torch.int64 else float("nan"))
        torch.cuda.synchronize()
        say("graph: replay", i)
        graph.replay()
        torch.cuda.synchronize()
        for k, (o, want) in enumerate(zip(outs, ref)):
            assert torch.equal(o, want), f"replay {i}: output {k} differs from the eager result"
