"""GPU parity: the general Mamba-1 kernels -- dstate up to 256 and
input-independent ([dim, dstate]) B / C -- forward and backward.

Forward against the C oracle (``oracle/scan_ref.c``, pinned to the torch
restatement of ``selective_scan_ref`` and to scalar float64 loops in
tests/test_oracle.py) on the same rounded inputs, at the reference test's
tolerances (external/mamba/tests/ops/test_selective_scan.py:43-45; fixture
tests/golden/mamba_scan_grid.json); backward against the float64
reverse-recurrence oracle at the reference's backward tolerances (:135-147:
an input-independent B / C is held to the weight tolerances rtolw / atolw,
an input-dependent one to rtol / atol). The grid's batch 2 x dim 4 is run at
dstate 8, 16, 32, 64 and 256 (the binding's limit, selective_scan.cpp:262)
in every B / C layout, and the reference's own N = 64 benchmark shape
(scripts/bench_external_kernels.py:140: B 8, D 384, L 512, N 64, fp16,
delta_softplus) forward and backward.
"""

import json
import os

import pytest
import torch

from gpu_util import gpu, need_gpu, say
from oracle import c_oracle, ops
from test_gpu_scan_bwd import NAMES

pytestmark = gpu
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GRID = json.load(open(os.path.join(GOLDEN, "mamba_scan_grid.json")))
ITYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
# layout -> (B input-independent, C input-independent, groups of the input-dependent ones)
LAYOUTS = {"var1": (False, False, 1), "var2": (False, False, 2), "constB": (True, False, 1),
           "constC": (False, True, 1), "constBC": (True, True, 1)}


def _inputs(batch, dim, dstate, seqlen, layout, itype, seed):
    cb, cc, groups = LAYOUTS[layout]
    g = torch.Generator().manual_seed(seed)
    A = -0.5 * torch.rand(dim, dstate, generator=g)
    # the reference test's draws: an input-independent B / C in the weight
    # type (fp32), an input-dependent one in the input type
    B = torch.randn(dim, dstate, generator=g) if cb else \
        torch.randn(batch, groups, dstate, seqlen, generator=g).to(itype)
    C = torch.randn(dim, dstate, generator=g) if cc else \
        torch.randn(batch, groups, dstate, seqlen, generator=g).to(itype)
    D = torch.randn(dim, generator=g)
    z = torch.randn(batch, dim, seqlen, generator=g).to(itype)
    bias = 0.5 * torch.rand(dim, generator=g)
    u = torch.randn(batch, dim, seqlen, generator=g).to(itype)
    delta = (0.5 * torch.rand(batch, dim, seqlen, generator=g)).to(itype)
    dout = torch.randn(batch, dim, seqlen, generator=g).to(itype)
    return u, delta, A, B, C, D, z, bias, dout


def _fwd(u, delta, A, B, C, D, z, bias, softplus):
    from kernels.hip.selective_scan import selective_scan_fn
    d = lambda t: None if t is None else t.to(DEV)
    out, last = selective_scan_fn(d(u), d(delta), d(A), d(B), d(C), d(D), d(z), d(bias), softplus, True)
    return out.cpu(), last.cpu()


def _grads(u, delta, A, B, C, D, z, bias, dout, softplus):
    from kernels.hip.selective_scan import selective_scan_fn
    leaves = [None if t is None else t.to(DEV).requires_grad_() for t in (u, delta, A, B, C, D, z, bias)]
    out = selective_scan_fn(*leaves[:5], D=leaves[5], z=leaves[6], delta_bias=leaves[7],
                            delta_softplus=softplus)
    out.backward(dout.to(DEV))
    return [None if t is None else t.grad.cpu() for t in leaves]


def _tols(itype, has_z, const_b, const_c):
    r, a = GRID["tolerances"][itype]
    rw, aw = 1e-3, 1e-3
    if has_z:
        rw, aw = max(rw, r), max(aw, a)
    return {"du": (2 * r, 2 * a), "ddelta": (5 * r, 10 * a), "dA": (rw, 5 * aw),
            "dB": (rw, aw) if const_b else (r, a), "dC": (rw, aw) if const_c else (r, a),
            "dD": (rw, aw), "dz": (rw, aw), "ddelta_bias": (rw, aw)}


def _check(got, ref, tols, inputs):
    for name, gv, rv, leaf in zip(NAMES, got, ref, inputs):
        if leaf is None:
            assert gv is None and rv is None, name
            continue
        assert gv.shape == leaf.shape and gv.dtype == leaf.dtype, name
        rt, at = tols[name]
        r = rv.to(leaf.dtype).double() if name in ("du", "ddelta", "dz") else rv
        err = (gv.double() - r).abs()
        bound = at + rt * r.abs()
        assert bool((err <= bound).all()), (name, float((err - bound).max()), float(err.max()))


@pytest.mark.parametrize("itype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("layout", list(LAYOUTS))
@pytest.mark.parametrize("dstate", [8, 16, 32, 64, 256])
@pytest.mark.parametrize("seqlen", [128, 2048])
def test_forward_reference_grid(itype, layout, dstate, seqlen):
    need_gpu()
    dt = ITYPES[itype]
    rtol, atol = GRID["tolerances"][itype]
    u, delta, A, B, C, D, z, bias, _ = _inputs(GRID["batch"], GRID["dim"], dstate, seqlen, layout,
                                               dt, dstate * 7 + seqlen)
    say("mamba wide fwd", itype, layout, dstate, seqlen)
    out, last = _fwd(u, delta, A, B, C, D, z, bias, True)
    ref, rlast = c_oracle.selective_scan(u, delta, A, B, C, D, z, bias, True)
    assert out.dtype == dt
    assert torch.allclose(out.float(), ref, rtol=rtol, atol=atol)
    assert torch.allclose(last, rlast, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("seqlen", GRID["seqlen"])
def test_forward_dstate64_full_seqlen_grid(seqlen):
    """The reference grid's every sequence length at dstate 64 (2-group B / C, fp32)."""
    need_gpu()
    rtol, atol = GRID["tolerances"]["float32"]
    u, delta, A, B, C, D, z, bias, _ = _inputs(2, 4, 64, seqlen, "var2", torch.float32, seqlen)
    say("mamba wide fwd seqlen", seqlen)
    out, last = _fwd(u, delta, A, B, C, D, z, bias, True)
    ref, rlast = c_oracle.selective_scan(u, delta, A, B, C, D, z, bias, True)
    assert torch.allclose(out, ref, rtol=rtol, atol=atol)
    assert torch.allclose(last, rlast, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("layout", list(LAYOUTS))
@pytest.mark.parametrize("dstate", [8, 32, 64, 256])
def test_backward_reference_grid(layout, dstate):
    need_gpu()
    if dstate == 8 and LAYOUTS[layout][:2] == (False, False):
        pytest.skip("dstate <= 16 with input-dependent B / C runs the specialised kernels "
                    "(tests/test_gpu_scan_bwd.py)")
    cb, cc, _ = LAYOUTS[layout]
    args = _inputs(GRID["batch"], GRID["dim"], dstate, 1024, layout, torch.float32, 500 + dstate)
    say("mamba wide bwd", layout, dstate)
    got = _grads(*args, softplus=True)
    u, delta, A, B, C, D, z, bias, dout = args
    ref = ops.selective_scan_bwd_ref(u, delta, A, B, C, dout, D, z, bias, True)
    _check(got, ref, _tols("float32", True, cb, cc), (u, delta, A, B, C, D, z, bias))


@pytest.mark.parametrize("itype", ["float16", "bfloat16"])
@pytest.mark.parametrize("layout,dstate,seqlen", [("var1", 48, 300), ("constBC", 24, 77),
                                                  ("constB", 256, 256)])
def test_backward_half_inputs_and_ragged(itype, layout, dstate, seqlen):
    """Half-precision inputs, partial state slots (dstate 24, 48), ragged
    sequence lengths, channels that do not fill a 16-channel workgroup."""
    need_gpu()
    cb, cc, _ = LAYOUTS[layout]
    u, delta, A, B, C, D, z, bias, dout = _inputs(2, 20, dstate, seqlen, layout, ITYPES[itype],
                                                  dstate + seqlen)
    say("mamba wide bwd half", itype, layout, dstate, seqlen)
    got = _grads(u, delta, A, B, C, D, z, bias, dout, True)
    ref = ops.selective_scan_bwd_ref(u, delta, A, B, C, dout, D, z, bias, True)
    _check(got, ref, _tols(itype, True, cb, cc), (u, delta, A, B, C, D, z, bias))


def test_reference_benchmark_shape_n64_forward_and_backward():
    """scripts/bench_external_kernels.py:140-156 of the reference: B 8, D 384,
    L 512, N 64, fp16 u / delta / B / C ([B, N, L]), fp32 A / D,
    delta_softplus, no gate, y.sum().backward()."""
    need_gpu()
    g = torch.Generator().manual_seed(140)
    Bn, Dn, L, N = 8, 384, 512, 64
    u = torch.randn(Bn, Dn, L, generator=g).half()
    delta = torch.randn(Bn, Dn, L, generator=g).half()
    A = -torch.rand(Dn, N, generator=g)
    Bm = torch.randn(Bn, N, L, generator=g).half()
    Cm = torch.randn(Bn, N, L, generator=g).half()
    Dv = torch.randn(Dn, generator=g)
    say("mamba N=64 reference benchmark shape")
    out, last = _fwd(u, delta, A, Bm, Cm, Dv, None, None, True)
    ref, rlast = c_oracle.selective_scan(u, delta, A, Bm, Cm, Dv, None, None, True)
    rtol, atol = GRID["tolerances"]["float16"]
    assert torch.allclose(out.float(), ref, rtol=rtol, atol=atol)
    assert torch.allclose(last, rlast, rtol=1e-4, atol=1e-3)
    got = _grads(u, delta, A, Bm, Cm, Dv, None, None, torch.ones_like(u), True)
    gref = ops.selective_scan_bwd_ref(u, delta, A, Bm, Cm, torch.ones_like(u), Dv, None, None, True)
    _check(got, gref, _tols("float16", False, False, False), (u, delta, A, Bm, Cm, Dv, None, None))


def test_wide_backward_deterministic_and_saved_states_path():
    """Bitwise-equal gradients over repeated runs, and the training path that
    keeps the forward's states gives every gradient but dz bitwise the same as
    the recompute path (dz within rounding)."""
    need_gpu()
    from kernels.hip import selective_scan as ss
    args = _inputs(2, 40, 64, 512, "constC", torch.bfloat16, 9)
    say("mamba wide bwd determinism")
    saved = ss.SAVE_STATES
    try:
        ss.set_save_states(True)
        runs = [_grads(*args, softplus=True) for _ in range(2)]
        ss.set_save_states(False)
        recomputed = _grads(*args, softplus=True)
    finally:
        ss.set_save_states(saved)
    for a, b in zip(runs[0], runs[1]):
        assert torch.equal(a, b)
    for name, a, b in zip(NAMES, runs[0], recomputed):
        if name == "dz":
            assert torch.allclose(a.float(), b.float(), rtol=1e-2, atol=1e-2)
        else:
            assert torch.equal(a, b), name


def test_wide_chunk_states_and_binding():
    """The binding's fwd at dstate 64 with an input-independent B: chunk states
    x against the float64 chunk-state oracle, out / out_z against the C oracle;
    its bwd returns dB in [dim, dstate] fp32."""
    need_gpu()
    from kernels.hip import selective_scan_cuda
    u, delta, A, B, C, D, z, bias, dout = _inputs(1, 16, 64, 4200, "constB", torch.float32, 12)
    d = lambda t: t.to(DEV)
    say("mamba wide binding")
    out, x, out_z = selective_scan_cuda.fwd(d(u), d(delta), d(A), d(B), d(C), d(D), d(z), d(bias), True)
    assert x.shape == (1, 16, 3, 128)
    xr = ops.selective_scan_chunk_states_ref(u, delta, A, B, bias, True)
    assert torch.allclose(x.cpu().double().view(1, 16, 3, 64, 2), xr, rtol=1e-4, atol=1e-5)
    ref_z, _ = c_oracle.selective_scan(u, delta, A, B, C, D, z, bias, True)
    ref, _ = c_oracle.selective_scan(u, delta, A, B, C, D, None, bias, True)
    assert torch.allclose(out.cpu(), ref, rtol=6e-4, atol=2e-3)
    assert torch.allclose(out_z.cpu(), ref_z, rtol=6e-4, atol=2e-3)
    res = selective_scan_cuda.bwd(d(u), d(delta), d(A), d(B), d(C), d(D), d(z), d(bias), d(dout),
                                  x, out, None, True, False)
    assert res[3].shape == (16, 64) and res[3].dtype == torch.float32
    gref = ops.selective_scan_bwd_ref(u, delta, A, B, C, dout, D, z, bias, True)
    assert torch.allclose(res[3].cpu().double(), gref[3], rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("itype", ["float32", "bfloat16"])
@pytest.mark.parametrize("layout", ["var1", "var2"])
@pytest.mark.parametrize("dstate", [24, 32, 48, 64])
def test_forward_rows_per_channel_kernels(itype, layout, dstate):
    """dstate 17-64 with input-dependent B / C on whole 64-step tiles runs the
    specialised forward with 2 or 4 lane rows per channel (dim 16: every
    channel tile whole): output and last state against the C oracle, with a
    gate, delta_bias and softplus, partial state slots at 24 and 48."""
    need_gpu()
    dt = ITYPES[itype]
    u, delta, A, B, C, D, z, bias, _ = _inputs(2, 16, dstate, 256, layout, dt, dstate + 3)
    say("mamba rows fwd", itype, layout, dstate)
    out, last = _fwd(u, delta, A, B, C, D, z, bias, True)
    ref, rlast = c_oracle.selective_scan(u, delta, A, B, C, D, z, bias, True)
    rtol, atol = GRID["tolerances"][itype]
    assert torch.allclose(out.float(), ref, rtol=rtol, atol=atol)
    assert torch.allclose(last, rlast, rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("dstate", [32, 64])
def test_rows_kernel_training_path_and_chunk_states(dstate):
    """The training forward on the rows kernels keeps its 16-step states, which
    the general backward then starts from: every gradient against the float64
    oracle, and the same gradients (dz within rounding) as the path that
    recomputes the states. The binding's chunk states x from the rows kernels
    against the chunk-state oracle over three 2048-step chunks."""
    need_gpu()
    from kernels.hip import selective_scan as ss
    from kernels.hip import selective_scan_cuda
    args = _inputs(2, 8, dstate, 512, "var1", torch.float32, 70 + dstate)
    say("mamba rows training path", dstate)
    saved = ss.SAVE_STATES
    try:
        ss.set_save_states(True)
        kept = _grads(*args, softplus=True)
        ss.set_save_states(False)
        recomputed = _grads(*args, softplus=True)
    finally:
        ss.set_save_states(saved)
    u, delta, A, B, C, D, z, bias, dout = args
    gref = ops.selective_scan_bwd_ref(u, delta, A, B, C, dout, D, z, bias, True)
    _check(kept, gref, _tols("float32", True, False, False), (u, delta, A, B, C, D, z, bias))
    for name, a, b in zip(NAMES, kept, recomputed):
        assert torch.allclose(a.double(), b.double(), rtol=1e-4, atol=1e-5), name
    u, delta, A, B, C, D, z, bias, _ = _inputs(1, 8, dstate, 4160, "var1", torch.float32, 5)
    d = lambda t: t.to(DEV)
    out, x, out_z = selective_scan_cuda.fwd(d(u), d(delta), d(A), d(B), d(C), d(D), d(z), d(bias), True)
    assert x.shape == (1, 8, 3, 2 * dstate)
    xr = ops.selective_scan_chunk_states_ref(u, delta, A, B, bias, True)
    assert torch.allclose(x.cpu().double().view(1, 8, 3, dstate, 2), xr, rtol=1e-4, atol=1e-5)
    ref_z, _ = c_oracle.selective_scan(u, delta, A, B, C, D, z, bias, True)
    assert torch.allclose(out_z.cpu(), ref_z, rtol=6e-4, atol=2e-3)
