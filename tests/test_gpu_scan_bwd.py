"""GPU parity: Mamba-1 selective-scan backward (ak_selective_scan_bwd).

Against the float64 reverse-recurrence oracle ``ops.selective_scan_bwd_ref``
(pinned to torch autograd of the forward oracle in tests/test_oracle.py) on
the same rounded inputs. Bars: the reference's backward tolerances
(external/mamba/tests/ops/test_selective_scan.py:43-49, :135-147) on its own
grid (tests/golden/mamba_scan_grid.json):
  du rtol 2r / atol 2a, ddelta 5r / 10a (both compared in the input dtype),
  dA rtolw / 5 atolw, dB and dC r / a (variable B / C), dD, dz, ddelta_bias
  rtolw / atolw,
with (r, a) = (6e-4, 2e-3) fp32, (3e-3, 5e-3) fp16, (3e-2, 5e-2) bf16 and
(rtolw, atolw) = (1e-3, 1e-3) raised to (r, a) when z is present. Every
gradient is bitwise reproducible (fixed summation order).
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


def _inputs(batch, dim, dstate, seqlen, groups, itype, seed, delta_dtype=None):
    g = torch.Generator().manual_seed(seed)
    A = -0.5 * torch.rand(dim, dstate, generator=g)
    Bs = (batch, groups, dstate, seqlen)
    B = torch.randn(*Bs, generator=g).to(itype)
    C = torch.randn(*Bs, generator=g).to(itype)
    D = torch.randn(dim, generator=g)
    z = torch.randn(batch, dim, seqlen, generator=g).to(itype)
    bias = 0.5 * torch.rand(dim, generator=g)
    u = torch.randn(batch, dim, seqlen, generator=g).to(itype)
    delta = (0.5 * torch.rand(batch, dim, seqlen, generator=g)).to(delta_dtype or itype)
    dout = torch.randn(batch, dim, seqlen, generator=g).to(itype)
    return u, delta, A, B, C, D, z, bias, dout


def _gpu_grads(u, delta, A, B, C, D, z, bias, dout, softplus):
    """Input gradients through selective_scan_fn's autograd (leaves on the GPU)."""
    from kernels.hip.selective_scan import selective_scan_fn
    leaves = [None if t is None else t.to(DEV).requires_grad_() for t in (u, delta, A, B, C, D, z, bias)]
    out = selective_scan_fn(*leaves[:5], D=leaves[5], z=leaves[6], delta_bias=leaves[7],
                            delta_softplus=softplus)
    out.backward(dout.to(DEV))
    return [None if t is None else t.grad.cpu() for t in leaves]


def _tols(itype, has_z):
    r, a = GRID["tolerances"][itype]
    rw, aw = 1e-3, 1e-3
    if has_z:
        rw, aw = max(rw, r), max(aw, a)
    return {"du": (2 * r, 2 * a), "ddelta": (5 * r, 10 * a), "dA": (rw, 5 * aw), "dB": (r, a),
            "dC": (r, a), "dD": (rw, aw), "dz": (rw, aw), "ddelta_bias": (rw, aw)}


def _check(got, ref, tols, inputs):
    for name, gv, rv, leaf in zip(NAMES, got, ref, inputs):
        if leaf is None:
            assert gv is None and rv is None, name
            continue
        assert gv.shape == leaf.shape and gv.dtype == leaf.dtype, name
        rt, at = tols[name]
        # du / ddelta / dz in the input dtype, as the reference test compares them
        r = rv.to(leaf.dtype).double() if name in ("du", "ddelta", "dz") else rv
        err = (gv.double() - r).abs()
        bound = at + rt * r.abs()
        assert bool((err <= bound).all()), (name, float((err - bound).max()), float(err.max()))


@pytest.mark.parametrize("itype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("groups", GRID["varBC_groups"])
@pytest.mark.parametrize("seqlen", GRID["seqlen"])
def test_reference_grid_backward(itype, groups, seqlen):
    need_gpu()
    dt = ITYPES[itype]
    args = _inputs(GRID["batch"], GRID["dim"], GRID["dstate"], seqlen, groups, dt, 1000 + seqlen + groups)
    say("mamba bwd grid", itype, groups, seqlen)
    got = _gpu_grads(*args, softplus=True)
    u, delta, A, B, C, D, z, bias, dout = args
    ref = ops.selective_scan_bwd_ref(u, delta, A, B, C, dout, D, z, bias, True)
    _check(got, ref, _tols(itype, True), (u, delta, A, B, C, D, z, bias))


@pytest.mark.parametrize("batch,dim,dstate,seqlen,groups,softplus,opts", [
    (1, 1, 1, 1, 1, True, "Dzb"), (3, 3, 5, 63, 1, False, ""), (2, 20, 16, 64, 1, True, "D"),
    (2, 40, 16, 100, 2, True, "zb"), (1, 16, 7, 129, 1, False, "Dz"), (2, 64, 16, 1000, 4, True, "Dzb"),
    (1, 33, 16, 257, 1, True, "b"), (2, 48, 16, 17, 3, False, "Dzb"), (1, 400, 16, 128, 1, True, "Dzb")])
def test_backward_shapes_and_options(batch, dim, dstate, seqlen, groups, softplus, opts):
    """Ragged tiles (seqlen and channels not multiples of 64 / 16), dstate
    below 16, several groups, each optional input present or absent; 400
    channels give 25 channel tiles, so the dB / dC tile sums take their 16-,
    8- and 1-partial loops."""
    need_gpu()
    u, delta, A, B, C, D, z, bias, dout = _inputs(batch, dim, dstate, seqlen, groups, torch.float32,
                                                  batch * 7 + dim + seqlen)
    D = D if "D" in opts else None
    z = z if "z" in opts else None
    bias = bias if "b" in opts else None
    say("mamba bwd shape", batch, dim, dstate, seqlen, groups, softplus, opts)
    got = _gpu_grads(u, delta, A, B, C, D, z, bias, dout, softplus)
    ref = ops.selective_scan_bwd_ref(u, delta, A, B, C, dout, D, z, bias, softplus)
    _check(got, ref, _tols("float32", z is not None), (u, delta, A, B, C, D, z, bias))


@pytest.mark.parametrize("itype,groups,softplus,opts", [("float32", 2, True, "Dzb"), ("bfloat16", 1, False, "D")])
def test_backward_wide_workgroups(itype, groups, softplus, opts):
    """Shapes whose reverse pass takes 32-channel workgroups (8 waves; batch x
    groups x channels / 32 = 256 workgroups, one per CU): every gradient
    against the oracle, and bitwise reproducible."""
    need_gpu()
    u, delta, A, B, C, D, z, bias, dout = _inputs(8, 1024, 16, 128, groups, ITYPES[itype], 77 + groups)
    D = D if "D" in opts else None
    z = z if "z" in opts else None
    bias = bias if "b" in opts else None
    say("mamba bwd 32-channel workgroups", itype, groups, softplus, opts)
    got = _gpu_grads(u, delta, A, B, C, D, z, bias, dout, softplus)
    again = _gpu_grads(u, delta, A, B, C, D, z, bias, dout, softplus)
    for a, b in zip(got, again):
        assert (a is None and b is None) or torch.equal(a, b)
    ref = ops.selective_scan_bwd_ref(u, delta, A, B, C, dout, D, z, bias, softplus)
    _check(got, ref, _tols(itype, z is not None), (u, delta, A, B, C, D, z, bias))


@pytest.mark.parametrize("itype", ["float16", "bfloat16"])
def test_backward_fp32_delta_and_bc(itype):
    """delta and B / C in fp32 with u in half precision (the forward's mixed
    layouts), 3-D B / C (dB / dC come back 3-D)."""
    need_gpu()
    dt = ITYPES[itype]
    u, delta, A, B, C, D, z, bias, dout = _inputs(2, 32, 16, 300, 1, dt, 3, delta_dtype=torch.float32)
    B3, C3 = B[:, 0].float(), C[:, 0].float()
    say("mamba bwd mixed dtypes", itype)
    got = _gpu_grads(u, delta, A, B3, C3, D, z, bias, dout, True)
    ref = ops.selective_scan_bwd_ref(u, delta, A, B3, C3, dout, D, z, bias, True)
    assert got[3].shape == B3.shape and got[4].shape == C3.shape
    _check(got, ref, _tols(itype, True), (u, delta, A, B3, C3, D, z, bias))


def test_backward_deterministic():
    need_gpu()
    args = _inputs(2, 64, 16, 1024, 1, torch.bfloat16, 5)
    say("mamba bwd determinism")
    runs = [_gpu_grads(*args, softplus=True) for _ in range(3)]
    for r in runs[1:]:
        for a, b in zip(runs[0], r):
            assert torch.equal(a, b)


def test_backward_delta_softplus_threshold():
    """delta + bias above 20: softplus is the identity there, so is its gradient."""
    need_gpu()
    u, delta, A, B, C, D, z, bias, dout = _inputs(1, 16, 16, 128, 1, torch.float32, 8)
    delta = delta + 19.8  # straddles the threshold with bias in [0, 0.5)
    A = A * 0.01          # keep exp(delta A) away from underflow
    say("mamba bwd softplus threshold")
    got = _gpu_grads(u, delta, A, B, C, D, z, bias, dout, True)
    ref = ops.selective_scan_bwd_ref(u, delta, A, B, C, dout, D, z, bias, True)
    _check(got, ref, _tols("float32", True), (u, delta, A, B, C, D, z, bias))


def test_c5_shape_backward():
    """The backward at C5's shape (bf16 u / z / B / C, fp32 delta, B4 D2048
    L4096 N16): per-channel gradients on a channel slice against the oracle
    run on that slice; dB / dC with dout zero outside a 48-channel slice that
    spans three channel tiles (the other channels then contribute exactly 0);
    bitwise reproducible."""
    need_gpu()
    import bench
    c = bench.gen_c5()
    g = torch.Generator().manual_seed(2)
    dout = torch.randn(c["u"].shape, generator=g).bfloat16()
    say("C5-shape mamba backward B4 L4096 D2048 N16")
    args = (c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["z"], None)
    got = _gpu_grads(*args, dout, False)
    again = _gpu_grads(*args, dout, False)
    for a, b in zip(got, again):
        assert (a is None and b is None) or torch.equal(a, b)
    tol = _tols("bfloat16", True)
    bsl, sl = slice(0, 1), slice(1000, 1008)
    ref = ops.selective_scan_bwd_ref(c["u"][bsl, sl], c["delta"][bsl, sl], c["A"][sl], c["B"][bsl],
                                     c["C"][bsl], dout[bsl, sl], c["D"][sl], c["z"][bsl, sl])
    for name, i in (("du", 0), ("ddelta", 1), ("dz", 6)):
        gv, rv = got[i][bsl, sl].double(), ref[i].to(got[i].dtype).double()
        rt, at = tol[name]
        assert bool(((gv - rv).abs() <= at + rt * rv.abs()).all()), name
    # dA / dD sum over the batch: compare the slice with all four sequences
    refb = ops.selective_scan_bwd_ref(c["u"][:, sl], c["delta"][:, sl], c["A"][sl], c["B"], c["C"],
                                      dout[:, sl], c["D"][sl], c["z"][:, sl])
    for name, i in (("dA", 2), ("dD", 5)):
        gv, rv = got[i][sl].double(), refb[i]
        rt, at = tol[name]
        assert bool(((gv - rv).abs() <= at + rt * rv.abs()).all()), name
    cs = slice(8, 56)
    dmask = torch.zeros_like(dout)
    dmask[:, cs] = dout[:, cs]
    part = _gpu_grads(*args, dmask, False)
    refc = ops.selective_scan_bwd_ref(c["u"][:, cs], c["delta"][:, cs], c["A"][cs], c["B"], c["C"],
                                      dmask[:, cs], c["D"][cs], c["z"][:, cs])
    for name, i in (("dB", 3), ("dC", 4)):
        gv, rv = part[i].double(), refc[i]
        rt, at = tol[name]
        assert bool(((gv - rv).abs() <= at + rt * rv.abs()).all()), name


def test_c5_backward_homogeneous_in_dout_bitwise():
    """Full C5 shape: every gradient is linear in dout and doubling dout is
    exact through the reverse recurrence, the sums over states, channels and
    the batch and the final rounding, so grads(2 dout) == 2 grads(dout) bit
    for bit (all outputs, all channels)."""
    need_gpu()
    import bench
    c = bench.gen_c5()
    g = torch.Generator().manual_seed(3)
    dout = torch.randn(c["u"].shape, generator=g).bfloat16()
    say("C5-shape mamba backward homogeneity in dout")
    args = (c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["z"], None)
    one = _gpu_grads(*args, dout, False)
    two = _gpu_grads(*args, 2 * dout, False)
    for a, b in zip(one, two):
        assert (a is None and b is None) or torch.equal(b, 2 * a)


@pytest.mark.parametrize("seqlen,fast", [(4196, False), (4096, True)])
def test_binding_fwd_chunk_states_and_prez(seqlen, fast):
    """kernels.hip.selective_scan_cuda.fwd on the GPU: ``out`` (before the
    gate), ``out_z`` and the chunk states ``x`` over 3 (ragged) or 2 chunks of
    2048 steps, against the oracles (float64 chunk states; the forward's
    tolerance of the reference grid). The state entries at rtol 1e-3 of the
    float64 prefix scan, the decay products at 1e-4 relative (they are
    exp2(A log2(e) sum delta') rather than a product of exps)."""
    need_gpu()
    from kernels.hip import selective_scan_cuda
    dim = 16 if fast else 5
    u, delta, A, B, C, D, z, bias, _ = _inputs(2, dim, 16, seqlen, 1, torch.float32, 21)
    A = A * 0.05  # keep the running decay products above fp32 underflow
    say("binding fwd chunk states", seqlen, fast)
    d = lambda t: t.to(DEV)
    out, x, out_z = selective_scan_cuda.fwd(d(u), d(delta), d(A), d(B), d(C), d(D), d(z), d(bias), True)
    nch = (seqlen + 2047) // 2048
    assert x.shape == (2, dim, nch, 32) and x.dtype == torch.float32
    xs = ops.selective_scan_chunk_states_ref(u, delta, A, B, bias, True).reshape(2, dim, nch, 32)
    xg = x.double().cpu()
    assert torch.allclose(xg[..., 1::2], xs[..., 1::2], rtol=1e-3, atol=1e-3)
    assert torch.allclose(xg[..., 0::2], xs[..., 0::2], rtol=1e-4, atol=1e-30)
    rt, at = GRID["tolerances"]["float32"]
    ref_prez = ops.selective_scan_ref(u, delta, A, B, C, D, None, bias, True)
    ref_z = ops.selective_scan_ref(u, delta, A, B, C, D, z, bias, True)
    assert torch.allclose(out.cpu(), ref_prez, rtol=rt, atol=at)
    assert torch.allclose(out_z.cpu(), ref_z, rtol=rt, atol=at)


def test_binding_bwd_matches_autograd(monkeypatch):
    """selective_scan_cuda.bwd (the reference binding's return list) gives the
    gradients selective_scan_fn's autograd gives when the latter recomputes
    the states too, bit for bit (same kernels), and writes dz into a caller
    buffer."""
    need_gpu()
    from kernels.hip import selective_scan, selective_scan_cuda
    monkeypatch.setattr(selective_scan, "SAVE_STATES", False)
    u, delta, A, B, C, D, z, bias, dout = _inputs(2, 32, 16, 512, 1, torch.bfloat16, 22)
    B3, C3 = B[:, 0], C[:, 0]
    say("binding bwd vs autograd")
    auto = _gpu_grads(u, delta, A, B3, C3, D, z, bias, dout, True)
    d = lambda t: t.to(DEV)
    out, x, out_z = selective_scan_cuda.fwd(d(u), d(delta), d(A), d(B3), d(C3), d(D), d(z), d(bias), True)
    dz_buf = torch.empty_like(d(z))
    res = selective_scan_cuda.bwd(d(u), d(delta), d(A), d(B3), d(C3), d(D), d(z), d(bias), d(dout), x, out,
                                  dz_buf, True, True)
    order = (0, 1, 2, 3, 4, 5, 7, 6)  # binding: du ddelta dA dB dC dD ddelta_bias dz
    for i, name in enumerate(NAMES):
        assert torch.equal(res[order[i]].cpu(), auto[i]), name
    assert res[7] is dz_buf
    assert torch.equal(res[8], out_z)


def test_backward_strided_views():
    """Inputs that are views (channel slices of wider tensors, B / C sliced
    from a wider state axis): the forward and backward take their strides as
    they are; gradients land in the viewed leaves' shapes."""
    need_gpu()
    u, delta, A, B, C, D, z, bias, dout = _inputs(2, 48, 16, 200, 1, torch.float32, 23)
    say("mamba bwd strided views")
    wide = lambda t: torch.cat([t, torch.zeros_like(t)], dim=1).to(DEV)
    uw, dw, zw = wide(u), wide(delta), wide(z)
    Bw = torch.cat([B, torch.zeros_like(B)], dim=2).to(DEV)   # [b, 1, 2n, l]
    Cw = torch.cat([C, torch.zeros_like(C)], dim=2).to(DEV)
    from kernels.hip.selective_scan import selective_scan_fn
    uw.requires_grad_(); dw.requires_grad_(); zw.requires_grad_(); Bw.requires_grad_(); Cw.requires_grad_()
    uv, dv, zv = uw[:, :48], dw[:, :48], zw[:, :48]
    Bv, Cv = Bw[:, :, :16], Cw[:, :, :16]
    assert not uv.is_contiguous() and not Bv.is_contiguous()
    Ad, Dd, bd = A.to(DEV).requires_grad_(), D.to(DEV).requires_grad_(), bias.to(DEV).requires_grad_()
    out = selective_scan_fn(uv, dv, Ad, Bv, Cv, Dd, zv, bd, True)
    out.backward(dout.to(DEV))
    ref = ops.selective_scan_bwd_ref(u, delta, A, B, C, dout, D, z, bias, True)
    got = [uw.grad[:, :48], dw.grad[:, :48], Ad.grad, Bw.grad[:, :, :16], Cw.grad[:, :, :16], Dd.grad,
           zw.grad[:, :48], bd.grad]
    _check([t.cpu() for t in got], ref, _tols("float32", True), (u, delta, A, B, C, D, z, bias))
    for t in (uw, dw, zw):
        assert float(t.grad[:, 48:].abs().max()) == 0.0
    assert float(Bw.grad[:, :, 16:].abs().max()) == 0.0 and float(Cw.grad[:, :, 16:].abs().max()) == 0.0


@pytest.mark.parametrize("itype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("batch,dim,seqlen,groups", [(2, 32, 512, 1), (1, 20, 300, 2), (2, 48, 1000, 1)])
def test_saved_states_backward_matches_recompute(monkeypatch, itype, batch, dim, seqlen, groups):
    """The training path (the forward keeps its states every 16 steps and its
    pre-gate output; the backward restarts from them) against the recompute
    path (the backward re-runs the forward): every gradient but dz bitwise
    equal, on the fast kernel's shapes and on ragged ones (generic kernel,
    2 groups); dz bitwise for fp32 and within one rounding of the stored
    pre-gate output for bf16. Both paths go through selective_scan_fn."""
    need_gpu()
    from kernels.hip import selective_scan
    args = _inputs(batch, dim, 16, seqlen, groups, itype, 31, delta_dtype=torch.float32)
    say("mamba bwd saved states vs recompute", itype, batch, dim, seqlen, groups)
    monkeypatch.setattr(selective_scan, "SAVE_STATES", True)
    saved = _gpu_grads(*args, softplus=True)
    monkeypatch.setattr(selective_scan, "SAVE_STATES", False)
    recomputed = _gpu_grads(*args, softplus=True)
    for name, a, b in zip(NAMES, saved, recomputed):
        if name == "dz" and itype != torch.float32:
            bound = 2.0 ** -7 * b.float().abs() + 1e-6 * float(b.float().abs().max())
            assert bool(((a.float() - b.float()).abs() <= bound).all()), name
        else:
            assert torch.equal(a, b), name


def test_saved_states_c_abi():
    """ak_selective_scan_fwd with a checkpoint buffer, then
    ak_selective_scan_bwd with and without it (no gate, so no out_prez is
    needed): identical gradients at the C5 channel / state layout."""
    need_gpu()
    from kernels.hip import _lib
    u, delta, A, B, C, D, z, bias, dout = (None if t is None else t.to(DEV) for t in
                                           _inputs(2, 64, 16, 1024, 1, torch.bfloat16, 33,
                                                   delta_dtype=torch.float32))
    say("mamba C-ABI checkpoints")
    out = torch.empty_like(u)
    ck = torch.full((2, 1024 // 16, 64, 16), float("nan"), device=DEV)
    _lib.selective_scan(u, delta, A, B, C, D, None, bias, out, None, True, checkpoints=ck)
    assert bool(torch.isfinite(ck).all())  # every block's state written
    assert bool((ck[:, 0] == 0).all())     # the state before step 0
    grads = []
    for use in (False, True):
        g = [torch.empty_like(u), torch.empty_like(delta), torch.empty_like(A), torch.empty_like(B),
             torch.empty_like(C), torch.empty_like(D), None, torch.empty_like(bias)]
        _lib.selective_scan_bwd(u, delta, A, B, C, D, None, bias, dout, *g[:6], g[6], g[7], True,
                                checkpoints=ck if use else None)
        grads.append(g)
    for name, a, b in zip(NAMES, *grads):
        assert (a is None and b is None) or torch.equal(a, b), name
