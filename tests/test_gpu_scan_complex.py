"""GPU parity: the Mamba-1 selective scan with complex A (ak_selective_scan_fwd
/ _bwd with a_dtype AK_DTYPE_C64).

Against the complex128 oracle (``ops.selective_scan_complex_ref`` and its
reverse-recurrence backward, pinned in tests/test_oracle.py by reduction to
the real scan, a brute-force double sum, a phase-rotation invariance, torch
autograd and central differences) on the same rounded inputs. Inputs follow
the reference test's complex branch (external/mamba/tests/ops/
test_selective_scan.py:55-75: A = -0.5 rand(dim, dstate) in complex64, B / C
real [batch, (groups,) dstate, 2 seqlen]), on its grid
(tests/golden/mamba_scan_grid.json) with its tolerances: out and
last_state (r, a) = (6e-4, 2e-3) fp32 / (3e-2, 5e-2) bf16; gradients as in
tests/test_gpu_scan_bwd.py (du 2r / 2a, ddelta 5r / 10a, dA rtolw / 5 atolw,
dB and dC r / a, dD, dz, ddelta_bias rtolw / atolw, with (rtolw, atolw) =
(1e-3, 1e-3) raised to (r, a) under a gate). Complex values are compared by
their real and imaginary parts. Every output is bitwise reproducible.
"""

import json
import os

import pytest
import torch

from gpu_util import gpu, need_gpu, say
from oracle import ops

pytestmark = gpu
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GRID = json.load(open(os.path.join(GOLDEN, "mamba_scan_grid.json")))
ITYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
NAMES = ("du", "ddelta", "dA", "dB", "dC", "dD", "dz", "ddelta_bias")


def _inputs(batch, dim, dstate, seqlen, groups, itype, seed, const_b=False, const_c=False):
    g = torch.Generator().manual_seed(seed)
    A = -0.5 * torch.complex(torch.rand(dim, dstate, generator=g), torch.rand(dim, dstate, generator=g))

    def bc(const):
        if const:
            return torch.complex(torch.randn(dim, dstate, generator=g), torch.randn(dim, dstate, generator=g))
        return torch.randn(batch, groups, dstate, 2 * seqlen, generator=g).to(itype)

    B, C = bc(const_b), bc(const_c)
    D = torch.randn(dim, generator=g)
    z = torch.randn(batch, dim, seqlen, generator=g).to(itype)
    bias = 0.5 * torch.rand(dim, generator=g)
    u = torch.randn(batch, dim, seqlen, generator=g).to(itype)
    delta = (0.5 * torch.rand(batch, dim, seqlen, generator=g)).to(itype)
    dout = torch.randn(batch, dim, seqlen, generator=g).to(itype)
    return u, delta, A, B, C, D, z, bias, dout


def _tols(itype, has_z):
    r, a = GRID["tolerances"][itype]
    rw, aw = 1e-3, 1e-3
    if has_z:
        rw, aw = max(rw, r), max(aw, a)
    return {"out": (r, a), "last": (r, a), "du": (2 * r, 2 * a), "ddelta": (5 * r, 10 * a),
            "dA": (rw, 5 * aw), "dB": (r, a), "dC": (r, a), "dD": (rw, aw), "dz": (rw, aw),
            "ddelta_bias": (rw, aw)}


def _close(name, got, ref, tol, like=None):
    if got.is_complex():
        got, ref = torch.view_as_real(got), torch.view_as_real(ref.to(torch.complex128))
    elif like is not None:  # compared in the input dtype, as the reference test does
        ref = ref.to(like).double()
    rt, at = tol
    err = (got.double() - ref.double()).abs()
    bound = at + rt * ref.double().abs()
    assert bool((err <= bound).all()), (name, float((err - bound).max()), float(err.max()))


def _run(u, delta, A, B, C, D, z, bias, dout, softplus, backward=True):
    from kernels.hip.selective_scan import selective_scan_fn
    leaves = [None if t is None else t.to(DEV).requires_grad_(backward) for t in (u, delta, A, B, C, D, z, bias)]
    out, last = selective_scan_fn(*leaves[:5], D=leaves[5], z=leaves[6], delta_bias=leaves[7],
                                  delta_softplus=softplus, return_last_state=True)
    grads = None
    if backward:
        out.backward(dout.to(DEV))
        grads = [None if t is None else t.grad.cpu() for t in leaves]
    return out.detach().cpu(), last.cpu(), grads


def _check_all(args, opts, softplus, itype, got):
    u, delta, A, B, C, D, z, bias, dout = args
    D = D if "D" in opts else None
    z = z if "z" in opts else None
    bias = bias if "b" in opts else None
    out, last, grads = got
    tol = _tols(itype, z is not None)
    ro, rl = ops.selective_scan_complex_ref(u, delta, A, B, C, D, z, bias, softplus, return_last_state=True)
    assert out.dtype == u.dtype and last.dtype == torch.complex64
    _close("out", out, ro, tol["out"], like=u.dtype)
    _close("last", last, rl, tol["last"])
    if grads is None:
        return
    ref = ops.selective_scan_complex_bwd_ref(u, delta, A, B, C, dout, D, z, bias, softplus)
    for name, gv, rv, leaf in zip(NAMES, grads, ref, (u, delta, A, B, C, D, z, bias)):
        if leaf is None:
            assert gv is None and rv is None, name
            continue
        assert gv.shape == leaf.shape and gv.dtype == leaf.dtype, name
        _close(name, gv, rv, tol[name], like=leaf.dtype if name in ("du", "ddelta", "dz") else None)


@pytest.mark.parametrize("itype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("groups", GRID["varBC_groups"])
@pytest.mark.parametrize("seqlen", GRID["seqlen"])
def test_complex_reference_grid(itype, groups, seqlen):
    """The reference test's grid with complex weights (its commented-out wtype
    complex64): forward, last state and every gradient."""
    need_gpu()
    dt = ITYPES[itype]
    args = _inputs(GRID["batch"], GRID["dim"], GRID["dstate"], seqlen, groups, dt, 2000 + seqlen + groups)
    say("complex scan grid", itype, groups, seqlen)
    u, delta, A, B, C, D, z, bias, dout = args
    got = _run(u, delta, A, B, C, D, z, bias, dout, True)
    _check_all(args, "Dzb", True, itype, got)


@pytest.mark.parametrize("batch,dim,dstate,seqlen,groups,softplus,opts,const", [
    (1, 1, 1, 1, 1, True, "Dzb", ""), (2, 6, 16, 37, 2, False, "D", ""), (2, 5, 64, 100, 1, True, "zb", ""),
    (1, 4, 65, 33, 1, True, "Dzb", ""), (1, 3, 130, 17, 1, False, "z", "B"), (1, 4, 256, 40, 2, True, "Dzb", ""),
    (2, 8, 16, 50, 1, True, "Dzb", "BC"), (1, 4, 8, 70, 1, False, "Db", "C"), (3, 12, 24, 129, 3, True, "Dz", "")])
def test_complex_shapes_and_options(batch, dim, dstate, seqlen, groups, softplus, opts, const):
    """Ragged tiles (seqlen not a multiple of 16, groups whose channels do not
    fill 4-channel workgroups), 1..4 state slots per lane (dstate up to 256),
    constant complex B / C, with and without gate, skip, bias and softplus."""
    need_gpu()
    args = _inputs(batch, dim, dstate, seqlen, groups, torch.float32, 71 + dstate + seqlen,
                   const_b="B" in const, const_c="C" in const)
    u, delta, A, B, C, D, z, bias, dout = args
    say("complex scan shape", batch, dim, dstate, seqlen, groups, softplus, opts, const)
    got = _run(u, delta, A, B, C, D if "D" in opts else None, z if "z" in opts else None,
               bias if "b" in opts else None, dout, softplus)
    _check_all(args, opts, softplus, "float32", got)


@pytest.mark.parametrize("itype,delta32,bc32", [("bfloat16", True, False), ("float16", False, True),
                                                ("bfloat16", True, True)])
def test_complex_mixed_dtypes(itype, delta32, bc32):
    """The forward's mixed layouts with complex weights: fp32 delta and / or
    fp32 B / C with half-precision u (each its own kernel instantiation)."""
    need_gpu()
    dt = ITYPES[itype]
    u, delta, A, B, C, D, z, bias, dout = _inputs(2, 8, 16, 90, 2, dt, 97)
    if delta32:
        delta = delta.float()
    if bc32:
        B, C = B.float(), C.float()
    say("complex scan mixed dtypes", itype, delta32, bc32)
    got = _run(u, delta, A, B, C, D, z, bias, dout, True)
    _check_all((u, delta, A, B, C, D, z, bias, dout), "Dzb", True, itype, got)


def test_complex_chunk_states_checkpoints_and_saved_backward():
    """Chunk states (two 2048-step chunks, the second ragged) against the
    oracle; the backward from the forward's complex checkpoints and pre-gate
    output equals the recomputing backward bit for bit, and both are bitwise
    reproducible."""
    need_gpu()
    from kernels.hip import _lib
    u, delta, A, B, C, D, z, bias, dout = (t.to(DEV) for t in
                                           _inputs(1, 4, 8, 2048 + 100, 1, torch.float32, 91))
    say("complex scan chunk states + checkpoints")
    out = torch.empty_like(u)
    prez = torch.empty_like(u)
    xs = torch.empty((1, 4, 2, 8, 2), dtype=torch.complex64, device=DEV)
    ck = torch.full((1, (2148 + 15) // 16, 4, 8), complex(float("nan"), 0.0), dtype=torch.complex64, device=DEV)
    _lib.selective_scan(u, delta, A, B, C, D, z, bias, out, None, True, out_prez=prez, chunk_states=xs,
                        checkpoints=ck)
    torch.cuda.synchronize()
    ref = ops.selective_scan_complex_chunk_states_ref(u.cpu(), delta.cpu(), A.cpu(), B.cpu(), bias.cpu(), True)
    _close("chunk_states", xs.cpu(), ref, (1e-4, 1e-4))
    assert bool(torch.isfinite(torch.view_as_real(ck)).all()) and bool((ck[:, 0] == 0).all())
    runs = []
    for saved in (True, False, True):
        g = [torch.empty_like(u), torch.empty_like(delta), torch.empty_like(A), torch.empty_like(B),
             torch.empty_like(C), torch.empty_like(D), torch.empty_like(z), torch.empty_like(bias)]
        _lib.selective_scan_bwd(u, delta, A, B, C, D, z, bias, dout, *g[:6], g[6], g[7], True,
                                checkpoints=ck if saved else None, out_prez=prez if saved else None)
        runs.append([t.cpu() for t in g])
    for name, a, b, c in zip(NAMES, *runs):
        assert torch.equal(a, b) and torch.equal(a, c), name


def test_complex_deterministic_and_empty():
    """Two runs give the same bits; zero steps give zero dA / dD / ddelta_bias
    and an empty output."""
    need_gpu()
    args = _inputs(2, 8, 32, 300, 2, torch.bfloat16, 93)
    say("complex scan determinism")
    u, delta, A, B, C, D, z, bias, dout = args
    a = _run(u, delta, A, B, C, D, z, bias, dout, True)
    b = _run(u, delta, A, B, C, D, z, bias, dout, True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    for x, y in zip(a[2], b[2]):
        assert torch.equal(x, y)
    say("complex scan zero steps")
    from kernels.hip import _lib
    e = [t[..., :0].contiguous().to(DEV) for t in (u, delta, z, dout)]
    Be = torch.zeros(2, 2, 32, 0, dtype=torch.bfloat16, device=DEV)
    dA = torch.full((8, 32), complex(1.0, 1.0), dtype=torch.complex64, device=DEV)
    dD = torch.ones(8, device=DEV)
    db = torch.ones(8, device=DEV)
    _lib.selective_scan_bwd(e[0], e[1], A.to(DEV), Be, Be, D.to(DEV), e[2], bias.to(DEV), e[3],
                            torch.empty_like(e[0]), torch.empty_like(e[1]), dA, torch.empty_like(Be),
                            torch.empty_like(Be), dD, torch.empty_like(e[0]), db, True)
    torch.cuda.synchronize()
    assert float(torch.view_as_real(dA).abs().max()) == 0.0
    assert float(dD.abs().max()) == 0.0 and float(db.abs().max()) == 0.0


def test_complex_binding_fwd_bwd():
    """kernels.hip.selective_scan_cuda with complex weights on the GPU: ``x``
    complex64 [batch, dim, n_chunks, 2 dstate], ``out`` / ``out_z``, and the
    backward's dA (complex), variable dB and constant dC against the oracle."""
    need_gpu()
    from kernels.hip import selective_scan_cuda
    u, delta, A, B, C, D, z, bias, dout = _inputs(2, 8, 16, 300, 2, torch.float32, 95, const_c=True)
    say("complex scan binding fwd / bwd")
    d = lambda t: t.to(DEV)
    out, x, out_z = selective_scan_cuda.fwd(d(u), d(delta), d(A), d(B), d(C), d(D), d(z), d(bias), True)
    assert x.shape == (2, 8, 1, 32) and x.dtype == torch.complex64
    tol = _tols("float32", True)
    xs = ops.selective_scan_complex_chunk_states_ref(u, delta, A, B, bias, True)
    _close("x", x.cpu(), xs.reshape(2, 8, 1, 32), (1e-4, 1e-4))
    _close("out", out.cpu(), ops.selective_scan_complex_ref(u, delta, A, B, C, D, None, bias, True),
           tol["out"], like=u.dtype)
    _close("out_z", out_z.cpu(), ops.selective_scan_complex_ref(u, delta, A, B, C, D, z, bias, True),
           tol["out"], like=u.dtype)
    res = selective_scan_cuda.bwd(d(u), d(delta), d(A), d(B), d(C), d(D), d(z), d(bias), d(dout), x, out,
                                  None, True, False)
    ref = ops.selective_scan_complex_bwd_ref(u, delta, A, B, C, dout, D, z, bias, True)
    for name, i in (("du", 0), ("ddelta", 1), ("dA", 2), ("dB", 3), ("dC", 4)):
        _close(name, res[i].cpu(), ref[i], tol[name], like=u.dtype if i < 2 else None)


def test_complex_strided_inputs():
    """u, delta, z and dout as channel-strided device views (every other
    channel of a wider tensor, last dim contiguous), through the C-ABI: the
    kernels take the batch / channel strides as given."""
    need_gpu()
    from kernels.hip import _lib
    u, delta, A, B, C, D, z, bias, dout = _inputs(2, 10, 16, 70, 1, torch.float32, 99)

    def strided(t):
        w = torch.stack([t, torch.full_like(t, float("nan"))], dim=2).reshape(t.shape[0], -1, t.shape[2])
        v = w.to(DEV)[:, ::2]
        assert not v.is_contiguous() and v.stride(1) == 2 * t.shape[2]
        return v

    us, ds, zs, gs = (strided(t) for t in (u, delta, z, dout))
    Ad, Bd, Cd, Dd, bd = (t.to(DEV) for t in (A, B, C, D, bias))
    say("complex scan strided inputs")
    out = torch.empty(u.shape, device=DEV)
    last = torch.empty((2, 10, 16), dtype=torch.complex64, device=DEV)
    _lib.selective_scan(us, ds, Ad, Bd, Cd, Dd, zs, bd, out, last, True)
    grads = [torch.empty(u.shape, device=DEV), torch.empty(u.shape, device=DEV), torch.empty_like(Ad),
             torch.empty_like(Bd), torch.empty_like(Cd), torch.empty_like(Dd), torch.empty(u.shape, device=DEV),
             torch.empty_like(bd)]
    _lib.selective_scan_bwd(us, ds, Ad, Bd, Cd, Dd, zs, bd, gs, *grads[:6], grads[6], grads[7], True)
    torch.cuda.synchronize()
    _check_all((u, delta, A, B, C, D, z, bias, dout), "Dzb", True, "float32",
               (out.cpu(), last.cpu(), [t.cpu() for t in grads]))
