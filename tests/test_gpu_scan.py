"""GPU parity: Mamba-1 selective scan and the diagonal recurrence.

Bars: the reference's selective-scan test grid and tolerances
(external/mamba/tests/ops/test_selective_scan.py:15-51, :43-45; fixture
tests/golden/mamba_scan_grid.json) against the C oracle on the same rounded
inputs; C5 at full size within rtol 1e-2 of the fp32 oracle (north star);
the reference's known-answer test for the diagonal scan.
"""

import json
import os

import pytest
import torch
import torch.nn.functional as F

from gpu_util import gpu, need_gpu, say
from oracle import c_oracle, ops

pytestmark = gpu
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GRID = json.load(open(os.path.join(GOLDEN, "mamba_scan_grid.json")))
ITYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def _inputs(batch, dim, dstate, seqlen, groups, itype, seed):
    g = torch.Generator().manual_seed(seed)
    A = -0.5 * torch.rand(dim, dstate, generator=g)
    Bs = (batch, groups, dstate, seqlen)
    B = torch.randn(*Bs, generator=g).to(itype)
    C = torch.randn(*Bs, generator=g).to(itype)
    D = torch.randn(dim, generator=g)
    z = torch.randn(batch, dim, seqlen, generator=g).to(itype)
    bias = 0.5 * torch.rand(dim, generator=g)
    u = torch.randn(batch, dim, seqlen, generator=g).to(itype)
    delta = (0.5 * torch.rand(batch, dim, seqlen, generator=g)).to(itype)
    return u, delta, A, B, C, D, z, bias


def _gpu(u, delta, A, B, C, D, z, bias, softplus, last=True):
    from kernels.hip.selective_scan import selective_scan_fn
    d = lambda t: None if t is None else t.to(DEV)
    r = selective_scan_fn(d(u), d(delta), d(A), d(B), d(C), d(D), d(z), d(bias), softplus, last)
    return (r[0].cpu(), r[1].cpu()) if last else r.cpu()


@pytest.mark.parametrize("itype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("groups", GRID["varBC_groups"])
@pytest.mark.parametrize("seqlen", GRID["seqlen"])
def test_reference_grid(itype, groups, seqlen):
    need_gpu()
    dt = ITYPES[itype]
    rtol, atol = GRID["tolerances"][itype]
    args = _inputs(GRID["batch"], GRID["dim"], GRID["dstate"], seqlen, groups, dt, seqlen + groups)
    say("mamba grid", itype, groups, seqlen)
    out, last = _gpu(*args, softplus=True)
    ref, rlast = c_oracle.selective_scan(*args, delta_softplus=True)
    assert out.dtype == dt
    assert torch.allclose(out.float(), ref, rtol=rtol, atol=atol)
    assert torch.allclose(last, rlast, rtol=rtol, atol=atol)


@pytest.mark.parametrize("batch,dim,dstate,seqlen,groups", [
    (1, 1, 1, 1, 1), (3, 3, 5, 63, 1), (2, 20, 16, 64, 1), (2, 40, 16, 100, 2), (1, 16, 7, 129, 1),
    (2, 64, 16, 1000, 4), (1, 33, 16, 257, 1)])
def test_shapes_and_options(batch, dim, dstate, seqlen, groups):
    need_gpu()
    u, delta, A, B, C, D, z, bias = _inputs(batch, dim, dstate, seqlen, groups, torch.bfloat16, dim * seqlen)
    say("mamba shapes", batch, dim, dstate, seqlen, groups)
    for softplus, zz, DD, bb in ((True, z, D, bias), (False, None, None, None)):
        out, last = _gpu(u, delta, A, B, C, DD, zz, bb, softplus)
        ref, rlast = c_oracle.selective_scan(u, delta, A, B, C, DD, zz, bb, softplus)
        assert torch.allclose(out.float(), ref, rtol=3e-2, atol=5e-2)
        assert torch.allclose(last, rlast, rtol=1e-4, atol=1e-4)
    # 3-D B / C and fp32 delta with bf16 u
    if groups == 1:
        out = _gpu(u, delta.float(), A, B[:, 0], C[:, 0], D, z, bias, True, last=False)
        ref, _ = c_oracle.selective_scan(u, delta.float(), A, B, C, D, z, bias, True)
        assert torch.allclose(out.float(), ref, rtol=3e-2, atol=5e-2)


@pytest.mark.parametrize("batch,dim,dstate,seqlen,groups,itype", [
    (2, 32, 16, 256, 1, "bfloat16"), (1, 64, 8, 512, 2, "float16"), (2, 16, 16, 128, 1, "float32"),
    (3, 48, 5, 64, 3, "bfloat16"), (1, 32, 16, 2048, 2, "bfloat16")])
def test_fast_path_shapes(batch, dim, dstate, seqlen, groups, itype):
    """Shapes on the vectorised whole-tile kernel (seqlen % 64 == 0, 16 | dim / groups)."""
    need_gpu()
    dt = ITYPES[itype]
    rtol, atol = GRID["tolerances"][itype]
    u, delta, A, B, C, D, z, bias = _inputs(batch, dim, dstate, seqlen, groups, dt, 3 * dim + seqlen)
    say("mamba fast path", batch, dim, dstate, seqlen, groups, itype)
    for softplus, zz, DD, bb in ((True, z, D, bias), (False, None, None, None), (False, z, D, None)):
        out, last = _gpu(u, delta, A, B, C, DD, zz, bb, softplus)
        ref, rlast = c_oracle.selective_scan(u, delta, A, B, C, DD, zz, bb, softplus)
        assert out.dtype == dt
        assert torch.allclose(out.float(), ref, rtol=rtol, atol=atol)
        assert torch.allclose(last, rlast, rtol=1e-4, atol=1e-4)
    if groups == 1:
        out = _gpu(u, delta.float(), A, B[:, 0], C[:, 0], D, z, bias, True, last=False)
        ref, _ = c_oracle.selective_scan(u, delta.float(), A, B, C, D, z, bias, True)
        assert torch.allclose(out.float(), ref, rtol=rtol, atol=atol)


def test_fast_and_generic_paths_agree():
    """The same scan through the whole-tile kernel (contiguous) and the generic
    kernel (a view with a row pitch that is not a multiple of 4 elements)."""
    need_gpu()
    u, delta, A, B, C, D, z, bias = _inputs(2, 32, 16, 320, 1, torch.bfloat16, 31)
    say("mamba fast vs generic")
    from kernels.hip.selective_scan import selective_scan_fn
    fast, lf = _gpu(u, delta, A, B, C, D, z, bias, True)
    pad = torch.zeros(2, 32, 321, dtype=torch.bfloat16, device=DEV)
    pad[..., :320] = u.to(DEV)
    uv = pad[..., :320]
    assert uv.stride(1) == 321
    d = lambda t: t.to(DEV)
    gen, lg = selective_scan_fn(uv, d(delta), d(A), d(B), d(C), d(D), d(z), d(bias), True, True)
    gen, lg = gen.cpu(), lg.cpu()
    ref, rl = c_oracle.selective_scan(u, delta, A, B, C, D, z, bias, True)
    assert torch.allclose(fast.float(), ref, rtol=3e-2, atol=5e-2)
    assert torch.allclose(gen.float(), ref, rtol=3e-2, atol=5e-2)
    assert torch.allclose(lf, lg, rtol=1e-5, atol=1e-5)
    # bf16 outputs of the two paths differ by at most one rounding step
    assert ((fast.float() - gen.float()).abs() <= 2 ** -7 * fast.float().abs() + 1e-6).all()


@pytest.mark.parametrize("itype,softplus,groups", [("bfloat16", False, 1), ("float32", True, 2),
                                                    ("float16", True, 1)])
def test_forward_variants_agree_bitwise(itype, softplus, groups):
    """The whole-tile forward is compiled in variants that fix its optional
    outputs: inference (a gate only), training (gate, pre-gate output and
    checkpoints), and a general one that tests them at run time (taken when
    chunk states are asked for, as the compiled binding's fwd does, or for a
    pre-gate output without checkpoints). They run the same arithmetic in the
    same order: every output has the same bits, fp16 outputs included (each
    value is rounded to fp32 before its storage type, as in the reference)."""
    need_gpu()
    from kernels.hip import _lib
    batch, dim, dstate, seqlen = 2, 64, 16, 512
    u, delta, A, B, C, D, z, bias = (t.to(DEV) for t in
                                     _inputs(batch, dim, dstate, seqlen, groups, ITYPES[itype], 41))
    say("mamba forward variants", itype, softplus, groups)

    def run(prez=False, ck=False, xs=False, gate=True):
        r = {"out": torch.empty_like(u), "last": torch.empty(batch, dim, dstate, device=DEV)}
        if prez:
            r["prez"] = torch.empty_like(u)
        if ck:
            r["ck"] = torch.empty(batch, seqlen // 16, dim, dstate, device=DEV)
        if xs:
            r["xs"] = torch.empty(batch, dim, (seqlen + 2047) // 2048, dstate, 2, device=DEV)
        _lib.selective_scan(u, delta, A, B, C, D, z if gate else None, bias, r["out"], r["last"], softplus,
                            out_prez=r.get("prez"), chunk_states=r.get("xs"), checkpoints=r.get("ck"))
        return r

    lean, train = run(), run(prez=True, ck=True)
    general, general_prez = run(prez=True, ck=True, xs=True), run(prez=True)
    ungated = run(prez=True, xs=True, gate=False)
    torch.cuda.synchronize()
    for k in ("out", "last"):
        assert torch.equal(lean[k], general[k]), k
        assert torch.equal(train[k], general[k]), k
    for k in ("prez", "ck"):
        assert torch.equal(train[k], general[k]), k
    assert torch.equal(general_prez["prez"], general["prez"])
    # without a gate the output is the pre-gate output, and the states are the gated call's
    assert torch.equal(ungated["out"], general["prez"]) and torch.equal(ungated["prez"], general["prez"])
    assert torch.equal(ungated["xs"], general["xs"]) and torch.equal(ungated["last"], general["last"])
    ref, rlast = c_oracle.selective_scan(u.cpu(), delta.cpu(), A.cpu(), B.cpu(), C.cpu(), D.cpu(), z.cpu(),
                                         bias.cpu(), softplus)
    rtol, atol = GRID["tolerances"][itype]
    assert torch.allclose(lean["out"].cpu().float(), ref, rtol=rtol, atol=atol)
    assert torch.allclose(lean["last"].cpu(), rlast, rtol=1e-4, atol=1e-4)


def test_whole_tile_forward_random_shapes():
    """Seeded random whole-tile shapes (seqlen a multiple of 64, channels per
    group a multiple of 16, dstate 1-16) with random dtypes and options,
    through the C-ABI: out and last_state against the C oracle at the
    reference grid's tolerances, and the inference / training / general
    variants of the producer / consumer forward bitwise equal to each other."""
    need_gpu()
    from kernels.hip import _lib
    rng = torch.Generator().manual_seed(2024)
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=rng))]
    for case in range(10):
        groups = pick([1, 1, 2, 4])
        batch, dim = pick([1, 2, 3]), 16 * groups * pick([1, 2, 3])
        dstate, seqlen = pick([1, 3, 8, 13, 16, 16]), 64 * pick([1, 2, 5, 8])
        itype = pick(["float32", "float16", "bfloat16"])
        softplus, use_bias, fp32_delta = pick([True, False]), pick([True, False]), pick([True, False])
        say("mamba random whole-tile forward", case, batch, dim, dstate, seqlen, groups, itype, softplus,
            use_bias, fp32_delta)
        u, delta, A, B, C, D, z, bias = _inputs(batch, dim, dstate, seqlen, groups, ITYPES[itype], 100 + case)
        if fp32_delta:
            delta = delta.float()
        bias = bias if use_bias else None
        dv = [t if t is None else t.to(DEV) for t in (u, delta, A, B, C, D, z, bias)]
        outs = []
        for prez, ck, xs in ((False, False, False), (True, True, False), (True, True, True)):
            out = torch.empty_like(dv[0])
            last = torch.empty(batch, dim, dstate, device=DEV)
            pz = torch.empty_like(dv[0]) if prez else None
            cks = torch.empty(batch, seqlen // 16, dim, dstate, device=DEV) if ck else None
            xss = torch.empty(batch, dim, (seqlen + 2047) // 2048, dstate, 2, device=DEV) if xs else None
            _lib.selective_scan(*dv, out, last, softplus, out_prez=pz, chunk_states=xss, checkpoints=cks)
            outs.append((out, last, pz, cks))
        torch.cuda.synchronize()
        for o in outs[1:]:
            assert torch.equal(o[0], outs[0][0]) and torch.equal(o[1], outs[0][1]), case
        assert torch.equal(outs[1][2], outs[2][2]) and torch.equal(outs[1][3], outs[2][3]), case
        ref, rlast = c_oracle.selective_scan(u, delta, A, B, C, D, z, bias, softplus)
        rtol, atol = GRID["tolerances"][itype]
        assert torch.allclose(outs[0][0].cpu().float(), ref, rtol=rtol, atol=atol), case
        assert torch.allclose(outs[0][1].cpu(), rlast, rtol=1e-3, atol=1e-3), case


def test_c5_full_size():
    need_gpu()
    import bench
    c = bench.gen_c5()
    say("C5 Mamba-1 scan B4 L4096 D2048 N16")
    out = _gpu(c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["z"], None, False, last=False)
    ref, _ = c_oracle.selective_scan(c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["z"])
    assert out.dtype == torch.bfloat16
    assert torch.allclose(out.float(), ref, rtol=1e-2, atol=1e-4)
    # the torch oracle (silu in fp32) agrees on a channel slice
    sl = slice(0, 8)
    tref = ops.selective_scan_ref(c["u"][:1, sl], c["delta"][:1, sl], c["A"][sl], c["B"][:1], c["C"][:1],
                                  c["D"][sl], c["z"][:1, sl])
    assert torch.allclose(out[:1, sl].float(), tref.float(), rtol=1e-2, atol=1e-4)


def test_c5_homogeneous_in_u_bitwise():
    """Full C5: the output is homogeneous of degree 1 in u, and scaling u by 2
    is exact at every step (delta u B, the state FMA, the sum over states,
    D u and the gate all scale by a power of two without new rounding), so
    scan(2u) must equal 2 scan(u) bit for bit."""
    need_gpu()
    import bench
    c = bench.gen_c5()
    say("C5 homogeneity in u")
    out = _gpu(c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["z"], None, False, last=False)
    out2 = _gpu(2 * c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["z"], None, False, last=False)
    assert torch.equal(out2, 2 * out)


def test_split_equivalence_on_gpu():
    """scan(L) == scan(L/2) continued from its last_state (closed-form invariant)."""
    need_gpu()
    u, delta, A, B, C, D, z, bias = _inputs(2, 32, 16, 512, 1, torch.float32, 77)
    say("mamba split equivalence")
    out, last = _gpu(u, delta, A, B, C, D, z, bias, True)
    a, s1 = _gpu(u[..., :256], delta[..., :256], A, B[..., :256], C[..., :256], D, z[..., :256], bias, True)
    ref2, s2 = c_oracle.selective_scan(u[..., 256:], delta[..., 256:], A, B[..., 256:], C[..., 256:], D,
                                       z[..., 256:], bias, True, initial_state=s1)
    assert torch.allclose(out[..., :256], a, rtol=1e-5, atol=1e-5)
    assert torch.allclose(out[..., 256:], ref2, rtol=1e-3, atol=1e-3)
    assert torch.allclose(last, s2, rtol=1e-3, atol=1e-4)


def test_deterministic():
    need_gpu()
    u, delta, A, B, C, D, z, bias = _inputs(2, 64, 16, 1024, 1, torch.bfloat16, 5)
    say("mamba determinism")
    outs = [_gpu(u, delta, A, B, C, D, z, bias, True)[0] for _ in range(3)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])


def test_diag_scan_known_answer_and_random():
    need_gpu()
    from kernels.hip.selective_scan import kernel_fn
    k = json.load(open(os.path.join(GOLDEN, "griffin_kat.json")))
    dA = torch.tensor(k["decay"]).view(1, 4, 1).to(DEV)
    dBx = torch.tensor(k["value"]).view(1, 4, 1).to(DEV)
    say("diag scan KAT")
    y = kernel_fn(dA, dBx, torch.ones_like(dA), torch.zeros(1, device=DEV), torch.zeros_like(dA))
    assert torch.allclose(y.view(-1).cpu(), torch.tensor(k["expected"]), rtol=1e-6)
    g = torch.Generator().manual_seed(9)
    shp = (8, 512, 384)
    dA = torch.sigmoid(torch.randn(*shp, generator=g))
    dBx = 0.1 * torch.randn(*shp, generator=g)
    C = torch.randn(*shp, generator=g)
    D = torch.randn(384, generator=g)
    x = torch.randn(*shp, generator=g)
    say("diag scan random", shp)
    y = kernel_fn(dA.to(DEV), dBx.to(DEV), C.to(DEV), D.to(DEV), x.to(DEV)).cpu()
    assert torch.allclose(y, ops.diag_scan_ref(dA, dBx, C, D, x), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("shp", [(8, 512, 384), (2, 1000, 33), (1, 1, 5), (3, 7, 1), (4, 4096, 64)])
def test_diag_scan_backward(shp):
    """ak_diag_scan_bwd against the float64 sequential backward
    (_torch_ops.py:346-386): fp32 bar 1e-5 relative (plus 1e-6 of the
    tensor's scale for entries that cancel)."""
    need_gpu()
    from kernels.hip.selective_scan_backward import kernel_fn
    g = torch.Generator().manual_seed(sum(shp))
    dA = torch.sigmoid(torch.randn(*shp, generator=g))
    dBx = 0.1 * torch.randn(*shp, generator=g)
    C = torch.randn(*shp, generator=g)
    D = torch.randn(shp[2], generator=g)
    x = torch.randn(*shp, generator=g)
    gy = torch.randn(*shp, generator=g)
    say("diag scan backward", shp)
    outs = kernel_fn(*(t.to(DEV) for t in (dA, dBx, C, D, x, gy)))
    refs = ops.diag_scan_bwd_ref(dA, dBx, C, D, x, gy)
    for got, ref in zip(outs, refs):
        got = got.double().cpu()
        bound = 1e-5 * ref.abs() + 1e-6 * float(ref.abs().max())
        assert bool(((got - ref).abs() <= bound).all()), float(((got - ref).abs() / bound).max())


@pytest.mark.parametrize("shp", [(1, 32, 3), (1, 33, 1), (3, 100, 7), (2, 1000, 33), (1, 5000, 8),
                                 (16, 1024, 384), (2, 31, 5), (512, 64, 384), (4, 2000, 48),
                                 (8, 256, 64), (2, 777, 1000)])
def test_diag_scan_chunk_plans(shp):
    """The diagonal scan's chunk plans at their edges, forward and backward
    against the float64 oracle: the smallest chunked lengths (32, 33 steps),
    a short last chunk (1000 = 58 x 17 + 14), the 64-chunk cap (5000 steps),
    AMADEUS's width, and shapes that stay sequential (31 steps; 2^17 lanes).
    Up to 1024 steps and from 16 channels the forward takes one launch and
    the backward its workgroup carry kernel and the 32-step sweep (AMADEUS: 32
    chunks of 32 steps; 1000 = 31 x 32 + 8 over 33 channels; 777 = 24 x 32 + 9
    steps over 1000 channels, whose last block of 32 holds 8; 256 and 64
    steps). Fewer channels or longer sequences run the chunked passes: chunks
    of up to 32 steps in the register kernels (1, 3 and 7 channels; 2000 = 62
    x 32 + 16 steps), longer ones streaming (5000 steps)."""
    need_gpu()
    from kernels.hip import selective_scan, selective_scan_backward
    g = torch.Generator().manual_seed(sum(shp) + 5)
    dA = torch.sigmoid(torch.randn(*shp, generator=g) + 2.0)
    dBx = 0.1 * torch.randn(*shp, generator=g)
    C = torch.randn(*shp, generator=g)
    D = torch.randn(shp[2], generator=g)
    x = torch.randn(*shp, generator=g)
    gy = torch.randn(*shp, generator=g)
    say("diag scan chunk plan", shp)
    y = selective_scan.kernel_fn(*(t.to(DEV) for t in (dA, dBx, C, D, x))).cpu().double()
    ref = ops.diag_scan_ref(dA.double(), dBx.double(), C.double(), D.double(), x.double())
    assert bool(((y - ref).abs() <= 1e-5 * ref.abs() + 1e-6 * float(ref.abs().max())).all())
    outs = selective_scan_backward.kernel_fn(*(t.to(DEV) for t in (dA, dBx, C, D, x, gy)))
    refs = ops.diag_scan_bwd_ref(dA, dBx, C, D, x, gy)
    for got, r in zip(outs, refs):
        got = got.double().cpu()
        bound = 1e-5 * r.abs() + 1e-6 * float(r.abs().max())
        assert bool(((got - r).abs() <= bound).all()), float(((got - r).abs() / bound).max())


def test_diag_scan_op_autograd_on_gpu():
    """torch.ops.autokernel.selective_scan backward on the GPU (the gfx950
    backward kernel) against the float64 sequential backward."""
    need_gpu()
    import kernels.hip._torch_ops  # noqa: F401
    g = torch.Generator().manual_seed(77)
    shp = (2, 300, 48)
    ins = [torch.sigmoid(torch.randn(*shp, generator=g)), 0.1 * torch.randn(*shp, generator=g),
           torch.randn(*shp, generator=g), torch.randn(48, generator=g), torch.randn(*shp, generator=g)]
    say("diag scan op autograd")
    dev = [t.to(DEV).requires_grad_() for t in ins]
    torch.ops.autokernel.selective_scan(*dev).pow(2).sum().backward()
    gy = 2 * ops.diag_scan_ref(*ins).double()  # d/dy of sum(y^2)
    refs = ops.diag_scan_bwd_ref(*ins, gy)
    for got, want in zip(dev, refs):
        assert torch.allclose(got.grad.double().cpu(), want, rtol=1e-4, atol=1e-4)


def test_softplus_accuracy_through_one_step():
    """delta_softplus on the GPU against float64 softplus: a one-step scan
    with A = 0, u = B = C = 1, D absent, no gate returns softplus(delta) times
    exact ones. Bar: 4e-6 relative (the kernel's exp2 argument x log2(e) is
    rounded to fp32: |x| log2(e) 2^-24 at |x| = 30), identity above 20,
    both fast and generic kernels (64 and 1 steps)."""
    need_gpu()
    x = torch.linspace(-30.0, 30.0, 4096)
    dim = x.numel()
    for seqlen in (1, 64):
        delta = x[None, :, None].expand(1, dim, seqlen).contiguous()
        u = torch.zeros(1, dim, seqlen)
        u[..., 0] = 1.0
        A = torch.zeros(dim, 1)
        B = torch.ones(1, 1, 1, seqlen)
        say("softplus accuracy", seqlen)
        out, _ = _gpu(u, delta, A, B, B, None, None, None, True)
        got = out[0, :, 0].double()
        xd = x.double()
        ref = torch.where(xd > 20, xd, torch.log1p(torch.exp(xd)))
        assert bool(((got - ref).abs() <= 4e-6 * ref.abs()).all()), float(((got - ref).abs() / ref.abs()).max())
