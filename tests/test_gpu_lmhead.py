"""GPU parity: fused lm-head + cross-entropy (MFMA GEMM + online logsumexp).

Bars: mean loss within 1e-3 relative of the fp32 oracle (north-star CE bar),
per-row logsumexp within 1e-4 relative, n_valid and ignore handling exact;
ChunkedLinearCrossEntropyLoss gradients within the reference's chunked-CE
test tolerances (test_chunked_ce.py:89-90: loss 1e-2, grads 5e-2 relative).
"""

import math

import pytest
import torch
import torch.nn.functional as F

from gpu_util import gpu, need_gpu, say
from oracle import ops

pytestmark = gpu
DEV = "cuda"


def _run(h, W, t, ignore_index=-100, softcap=0.0, ls=0.0):
    from kernels.hip.chunked_linear_cross_entropy import lmhead_ce_forward
    return lmhead_ce_forward(h.to(DEV), W.to(DEV), t.to(DEV), ignore_index, return_losses=True,
                             softcap=softcap, label_smoothing=ls)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
# Shapes cover every tile-kernel variant: matrices under 256 rows (clamped
# re-reads), vocab % 128 != 0 (element-wise tail mask), vocab % 128 == 0 but
# not % 256 (shifted tail tile skipping a whole 128-row half), token tails,
# and 1, 2, 3 and more 64-wide K blocks per tile (the LDS ring then looks
# up to three tiles ahead). Vocab 70,000 has more tile partials per row than
# the row kernel loads at once (its looped merge).
@pytest.mark.parametrize("n,vocab,d", [(1, 1, 64), (5, 300, 64), (300, 1000, 128), (257, 4097, 768),
                                       (512, 50304, 768), (1000, 256, 192), (300, 1152, 128),
                                       (700, 640, 64), (260, 384, 64), (2000, 2432, 192), (64, 70000, 64)])
def test_lmhead_ce_matches_oracle(dtype, n, vocab, d):
    need_gpu()
    g = torch.Generator().manual_seed(n * 7 + vocab)
    h = torch.randn(n, d, generator=g).to(dtype)
    W = (0.05 * torch.randn(vocab, d, generator=g)).to(dtype)
    t = torch.randint(0, vocab, (n,), generator=g)
    t[: max(0, n // 10)] = -100
    say("lmhead_ce", dtype, n, vocab, d)
    loss, lse, nv, losses = _run(h, W, t)
    rloss, rlse, rlosses = ops.lmhead_ce_ref(h, W, t)
    assert int(nv) == int((t != -100).sum())
    assert torch.allclose(lse.double().cpu(), rlse.double(), rtol=1e-4, atol=1e-4)
    assert torch.allclose(losses.double().cpu(), rlosses.double(), rtol=1e-3, atol=1e-3)
    assert abs(float(loss) - float(rloss)) <= 1e-3 * abs(float(rloss)) + 1e-6
    assert bool((losses.cpu()[t == -100] == 0).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cap", [30.0, 2.0])
@pytest.mark.parametrize("n,vocab,d", [(5, 300, 64), (257, 4097, 768), (300, 1152, 128), (700, 640, 64),
                                       (512, 50304, 768)])
def test_lmhead_ce_softcap_matches_oracle(dtype, cap, n, vocab, d):
    """The logit softcap in the fused kernel (every tile-kernel variant)
    against the streamed fp32 oracle with the same softcap; cap 2 saturates
    most logits (weights scaled up), cap 30 is the reference's usual value."""
    need_gpu()
    g = torch.Generator().manual_seed(n * 5 + vocab)
    h = torch.randn(n, d, generator=g).to(dtype)
    W = ((0.5 if cap < 10 else 0.05) * torch.randn(vocab, d, generator=g)).to(dtype)
    t = torch.randint(0, vocab, (n,), generator=g)
    t[: max(0, n // 10)] = -100
    say("lmhead_ce softcap", dtype, cap, n, vocab, d)
    loss, lse, nv, losses = _run(h, W, t, softcap=cap)
    rloss, rlse, rlosses = ops.lmhead_ce_ref(h, W, t, softcap=cap)
    assert int(nv) == int((t != -100).sum())
    assert torch.allclose(lse.double().cpu(), rlse.double(), rtol=1e-4, atol=1e-4)
    assert torch.allclose(losses.double().cpu(), rlosses.double(), rtol=1e-3, atol=1e-3)
    assert abs(float(loss) - float(rloss)) <= 1e-3 * abs(float(rloss)) + 1e-6
    assert bool((losses.cpu()[t == -100] == 0).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cap,ls", [(0.0, 0.1), (30.0, 0.1), (0.0, 1.0), (4.0, 0.3)])
@pytest.mark.parametrize("n,vocab,d", [(5, 300, 64), (257, 4097, 768), (300, 1152, 128), (700, 640, 64),
                                       (512, 50304, 768)])
def test_lmhead_ce_label_smoothing_matches_oracle(dtype, cap, ls, n, vocab, d):
    """Label smoothing in the fused forward (every tile-kernel variant, with
    and without a softcap) against the streamed fp32 oracle: lse to 1e-4,
    per-row losses and the mean to 1e-3 (the per-tile logit sums are fp32)."""
    need_gpu()
    g = torch.Generator().manual_seed(n * 11 + vocab)
    h = torch.randn(n, d, generator=g).to(dtype)
    W = ((0.3 if 0 < cap < 10 else 0.05) * torch.randn(vocab, d, generator=g)).to(dtype)
    t = torch.randint(0, vocab, (n,), generator=g)
    t[: max(0, n // 10)] = -100
    say("lmhead_ce label smoothing", dtype, cap, ls, n, vocab, d)
    loss, lse, nv, losses = _run(h, W, t, softcap=cap, ls=ls)
    rloss, rlse, rlosses = ops.lmhead_ce_ref(h, W, t, softcap=cap, label_smoothing=ls)
    assert int(nv) == int((t != -100).sum())
    assert torch.allclose(lse.double().cpu(), rlse.double(), rtol=1e-4, atol=1e-4)
    assert torch.allclose(losses.double().cpu(), rlosses.double(), rtol=1e-3, atol=1e-3)
    assert abs(float(loss) - float(rloss)) <= 1e-3 * abs(float(rloss)) + 1e-6
    assert bool((losses.cpu()[t == -100] == 0).all())


def test_lmhead_all_ignored_and_bad_targets():
    need_gpu()
    g = torch.Generator().manual_seed(1)
    h = torch.randn(64, 128, generator=g).bfloat16()
    W = (0.05 * torch.randn(500, 128, generator=g)).bfloat16()
    say("lmhead all ignored")
    loss, lse, nv, losses = _run(h, W, torch.full((64,), -100))
    assert float(loss) == 0.0 and int(nv) == 0
    t = torch.randint(0, 500, (64,), generator=g)
    t[3] = 500
    loss, lse, nv, losses = _run(h, W, t)
    assert math.isnan(float(losses[3])) and math.isnan(float(loss))
    # h = 0: every logit is 0, lse = log V exactly up to rounding, loss = log V
    loss, lse, nv, losses = _run(torch.zeros(16, 64).bfloat16(), W[:, :64].contiguous(), torch.arange(16))
    assert torch.allclose(lse.cpu(), torch.full((16,), math.log(500)), rtol=1e-6)
    assert abs(float(loss) - math.log(500)) < 1e-5


_C4_ORACLE = {}
# bf16 round to nearest: within 2^-8 of the value (8 significant bits), with
# 1% room for the fp32 arithmetic before the rounding
_U8 = 1.01 * 2.0 ** -8


def _c4_oracle(c):
    """float64 oracle (loss, lse, per-row losses) of the whole C4 problem,
    computed once per process (about 630 GFLOP on the host)."""
    if not _C4_ORACLE:
        loss, lse, losses = ops.lmhead_ce_ref(c["h"], c["W"], c["t"], dtype=torch.float64)
        _C4_ORACLE.update(loss=loss, lse=lse, losses=losses)
    return _C4_ORACLE["loss"], _C4_ORACLE["lse"], _C4_ORACLE["losses"]


def test_c4_full_size():
    """C4 against the float64 oracle on all 8,192 rows: logsumexp, per-row
    losses (zero on ignored rows), the mean, and the count of valid rows."""
    need_gpu()
    import bench
    c = bench.gen_c4()
    say("C4 lm-head + CE bf16 [8192, 768] x [50304, 768]")
    loss, lse, nv, losses = _run(c["h"], c["W"], c["t"])
    t = c["t"]
    valid = t != -100
    assert int(nv) == int(valid.sum()) == 8192 - 409
    rloss, rlse, rl = _c4_oracle(c)
    lse_c, losses_c = lse.cpu().double(), losses.cpu().double()
    assert torch.allclose(lse_c, rlse, rtol=2e-5, atol=0.0), float((lse_c - rlse).abs().max())
    assert torch.allclose(losses_c, rl, rtol=2e-5, atol=2e-5), float((losses_c - rl).abs().max())
    assert bool((losses.cpu()[~valid] == 0).all())
    assert abs(float(loss) - float(rloss)) <= 1e-5 * abs(float(rloss)), (float(loss), float(rloss))
    # deterministic: same bits on a second call
    loss2, lse2, _, _ = _run(c["h"], c["W"], c["t"])
    assert torch.equal(lse2, lse) and torch.equal(loss2, loss)


def test_c4_token_permutation_equivariance_bitwise():
    """Full C4: each token's logits, logsumexp and loss are computed by the same
    operations in the same order wherever the token sits (every token tile is
    whole at 8192 tokens), so permuting the tokens permutes lse and the per-row
    losses bit for bit."""
    need_gpu()
    import bench
    c = bench.gen_c4()
    perm = torch.randperm(8192, generator=torch.Generator().manual_seed(9))
    _, lse, _, losses = _run(c["h"], c["W"], c["t"])
    _, lse_p, _, losses_p = _run(c["h"][perm], c["W"], c["t"][perm])
    assert torch.equal(lse_p.cpu(), lse.cpu()[perm])
    assert torch.equal(losses_p.cpu(), losses.cpu()[perm])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("softcap,ls,zw", [(0.0, 0.0, 0.0), (0.0, 0.0, 1e-4), (20.0, 0.0, 0.0),
                                           (30.0, 0.0, 1e-4), (0.0, 0.1, 0.0), (30.0, 0.1, 1e-4)])
def test_chunked_linear_ce_fwd_bwd(dtype, softcap, ls, zw):
    need_gpu()
    from kernels.hip.chunked_linear_cross_entropy import ChunkedLinearCrossEntropyLoss
    g = torch.Generator().manual_seed(3)
    B, T, D, V = 4, 128, 256, 3000
    h0 = torch.randn(B, T, D, generator=g)
    W0 = 0.05 * torch.randn(V, D, generator=g)
    t = torch.randint(0, V, (B, T), generator=g)
    t[0, :10] = -100
    h = h0.to(dtype).to(DEV).requires_grad_()
    W = W0.to(dtype).to(DEV).requires_grad_()
    say("chunked linear ce", dtype, softcap, ls, zw)
    loss = ChunkedLinearCrossEntropyLoss(chunk_size=100, softcap=softcap, label_smoothing=ls,
                                         z_loss_weight=zw)(h, W, t.to(DEV))
    loss.backward()
    hr = h0.to(dtype).double().requires_grad_()
    Wr = W0.to(dtype).double().requires_grad_()
    logits = hr.reshape(-1, D) @ Wr.t()
    if softcap > 0:
        logits = softcap * torch.tanh(logits / softcap)
    ref = F.cross_entropy(logits, t.reshape(-1), label_smoothing=ls)
    ref.backward()
    if zw > 0:
        valid = (t.reshape(-1) != -100).double()
        ref = ref + zw * ((torch.logsumexp(logits.detach(), -1) * valid) ** 2).sum() / valid.sum()
    assert abs(float(loss) - float(ref)) <= 1e-2 * abs(float(ref))
    for got, want in ((h.grad, hr.grad), (W.grad, Wr.grad)):
        rel = float((got.double().cpu() - want).norm() / want.norm())
        assert rel < 5e-2, rel


# ---------------------------------------------------------------------------
# Fused backward: dL/dlogits from the matrix cores, then two GEMMs
# ---------------------------------------------------------------------------

def _dz_ref(h, W, t, lse, scale, ignore_index=-100, softcap=0.0, ls=0.0):
    """float64 softmax(h W^T) - onehot, times scale, from the GPU forward's lse
    (through the softcap z' = c tanh(z / c), times 1 - tanh^2, when c > 0;
    label smoothing a: softmax - (1 - a) onehot - a / V)."""
    z = h.double() @ W.double().t()
    dcap = 1.0
    if softcap > 0:
        th = torch.tanh(z / softcap)
        z, dcap = softcap * th, 1 - th * th
    p = torch.exp(z - lse.double()[:, None]) - ls / W.shape[0]
    tc = t.clamp(min=0)
    p[torch.arange(len(t)), tc] -= 1.0 - ls
    p = p * scale * dcap
    p[t == ignore_index] = 0.0
    return p


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,vocab,d", [(5, 300, 64), (300, 1000, 128), (257, 4097, 768), (1000, 256, 192),
                                       (300, 1152, 128), (2000, 2432, 192), (512, 50304, 768)])
def test_lmhead_ce_grad_logits(dtype, n, vocab, d):
    """ak_lmhead_ce_bwd against float64 softmax - onehot: each entry within one
    rounding of the element type (plus 1e-6 of the scale, and fp16's subnormal
    half-spacing); ignored rows exactly 0."""
    need_gpu()
    from kernels.hip import _lib
    g = torch.Generator().manual_seed(n + vocab)
    h = torch.randn(n, d, generator=g).to(dtype)
    W = (0.05 * torch.randn(vocab, d, generator=g)).to(dtype)
    t = torch.randint(0, vocab, (n,), generator=g)
    t[: max(0, n // 10)] = -100
    say("lmhead_ce grad logits", dtype, n, vocab, d)
    loss, lse, nv, _ = _run(h, W, t)
    denom = nv.to(torch.float32).clamp(min=1.0).reshape(1)
    gl = torch.tensor([0.75], device=DEV)
    ldv = vocab + 3  # a padded pitch: the padding must stay untouched
    dz = torch.full((n, ldv), 5.0, dtype=dtype, device=DEV)
    _lib.lmhead_ce_bwd(h.to(DEV), W.to(DEV), t.to(DEV), lse, gl, denom, dz, -100)
    scale = 0.75 / float(denom)
    ref = _dz_ref(h, W, t, lse.cpu(), scale)
    got = dz[:, :vocab].double().cpu()
    err = (got - ref).abs()
    eps = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    # fp16 entries below 2^-14 are subnormal: absolute spacing 2^-24
    floor = 1e-6 * scale + (2.0 ** -25 if dtype == torch.float16 else 0.0)
    assert bool((err <= eps * ref.abs() + floor).all()), float((err / (eps * ref.abs() + floor)).max())
    assert bool((got[t == -100] == 0).all())
    if ldv > vocab:
        assert bool((dz[:, vocab:].float().cpu() == 5.0).all())  # row padding untouched


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,vocab,d", [(5, 300, 64), (257, 4097, 768), (300, 1152, 128), (512, 50304, 768)])
def test_lmhead_ce_grad_logits_softcap(dtype, n, vocab, d):
    """dL/dlogits through the softcap (cap 3: logits up to about 3 cap, so
    1 - tanh^2 spans [0.01, 1]) against float64, to one rounding of the element
    type plus 2e-6 of the scale (the fp32 arithmetic of q, r and exp)."""
    need_gpu()
    from kernels.hip import _lib
    cap = 3.0
    g = torch.Generator().manual_seed(n * 3 + vocab)
    h = torch.randn(n, d, generator=g).to(dtype)
    W = (0.3 * torch.randn(vocab, d, generator=g) / math.sqrt(d / 64)).to(dtype)
    t = torch.randint(0, vocab, (n,), generator=g)
    t[: max(0, n // 10)] = -100
    say("lmhead_ce grad logits softcap", dtype, n, vocab, d)
    loss, lse, nv, _ = _run(h, W, t, softcap=cap)
    denom = nv.to(torch.float32).clamp(min=1.0).reshape(1)
    gl = torch.tensor([0.75], device=DEV)
    dz = torch.empty((n, vocab), dtype=dtype, device=DEV)
    _lib.lmhead_ce_bwd(h.to(DEV), W.to(DEV), t.to(DEV), lse, gl, denom, dz, -100, cap)
    scale = 0.75 / float(denom)
    ref = _dz_ref(h, W, t, lse.cpu(), scale, softcap=cap)
    got = dz.double().cpu()
    err = (got - ref).abs()
    eps = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    floor = 2e-6 * scale + (2.0 ** -25 if dtype == torch.float16 else 0.0)
    assert bool((err <= eps * ref.abs() + floor).all()), float((err / (eps * ref.abs() + floor)).max())
    assert bool((got[t == -100] == 0).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cap,ls", [(0.0, 0.1), (3.0, 0.2)])
@pytest.mark.parametrize("n,vocab,d", [(5, 300, 64), (257, 4097, 768), (300, 1152, 128), (512, 50304, 768)])
def test_lmhead_ce_grad_logits_label_smoothing(dtype, cap, ls, n, vocab, d):
    """dL/dlogits with label smoothing (and a softcap) against float64, to one
    rounding of the element type plus 2e-6 of the scale."""
    need_gpu()
    from kernels.hip import _lib
    g = torch.Generator().manual_seed(n * 13 + vocab)
    h = torch.randn(n, d, generator=g).to(dtype)
    W = ((0.3 / math.sqrt(d / 64) if cap else 0.05) * torch.randn(vocab, d, generator=g)).to(dtype)
    t = torch.randint(0, vocab, (n,), generator=g)
    t[: max(0, n // 10)] = -100
    say("lmhead_ce grad logits label smoothing", dtype, cap, ls, n, vocab, d)
    loss, lse, nv, _ = _run(h, W, t, softcap=cap, ls=ls)
    denom = nv.to(torch.float32).clamp(min=1.0).reshape(1)
    gl = torch.tensor([0.75], device=DEV)
    dz = torch.empty((n, vocab), dtype=dtype, device=DEV)
    _lib.lmhead_ce_bwd(h.to(DEV), W.to(DEV), t.to(DEV), lse, gl, denom, dz, -100, cap, ls)
    scale = 0.75 / float(denom)
    ref = _dz_ref(h, W, t, lse.cpu(), scale, softcap=cap, ls=ls)
    got = dz.double().cpu()
    err = (got - ref).abs()
    eps = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    floor = 2e-6 * scale + (2.0 ** -25 if dtype == torch.float16 else 0.0)
    assert bool((err <= eps * ref.abs() + floor).all()), float((err / (eps * ref.abs() + floor)).max())
    assert bool((got[t == -100] == 0).all())


def test_c4_full_size_softcap():
    """C4 with the reference's usual logit softcap (30): forward on a row
    subset against the oracle, the mean from GPU lse and exact capped target
    logits; backward rows of dlogits against float64; deterministic."""
    need_gpu()
    import bench
    from kernels.hip import _lib
    c = bench.gen_c4()
    say("C4 lm-head + CE with softcap 30")
    loss, lse, nv, losses = _run(c["h"], c["W"], c["t"], softcap=30.0)
    loss2, lse2, _, _ = _run(c["h"], c["W"], c["t"], softcap=30.0)
    assert torch.equal(lse, lse2) and torch.equal(loss, loss2)
    t = c["t"]
    valid = t != -100
    idx = torch.randperm(8192, generator=torch.Generator().manual_seed(3))[:256].sort().values
    _, rlse, rl = ops.lmhead_ce_ref(c["h"][idx], c["W"], t[idx], softcap=30.0)
    assert torch.allclose(lse.cpu()[idx].double(), rlse.double(), rtol=1e-4)
    assert torch.allclose(losses.cpu()[idx].double(), rl.double(), rtol=1e-3, atol=1e-3)
    xt = 30.0 * torch.tanh((c["h"].float() * c["W"][t.clamp(min=0)].float()).sum(-1).double() / 30.0)
    ref_loss = ((lse.cpu().double() - xt) * valid.double()).sum() / valid.sum()
    assert abs(float(loss) - float(ref_loss)) <= 1e-3 * abs(float(ref_loss))
    denom = nv.to(torch.float32).clamp(min=1.0).reshape(1)
    one = torch.ones(1, device=DEV)
    dz = torch.empty(8192, 50304, dtype=torch.bfloat16, device=DEV)
    _lib.lmhead_ce_bwd(c["h"].to(DEV), c["W"].to(DEV), t.to(DEV), lse, one, denom, dz, -100, 30.0)
    scale = 1.0 / float(denom)
    ref = _dz_ref(c["h"][idx], c["W"], t[idx], lse.cpu()[idx], scale, softcap=30.0)
    got = dz[idx.to(DEV)].double().cpu()
    assert bool(((got - ref).abs() <= 2.0 ** -8 * ref.abs() + 2e-6 * scale).all())


def test_lmhead_ce_grad_logits_pitch_fallback():
    """A grad_logits pitch that is a multiple of 4 but not of 8 takes the
    element-wise store path; the result is the same as the vector path's."""
    need_gpu()
    from kernels.hip import _lib
    g = torch.Generator().manual_seed(21)
    h = torch.randn(600, 128, generator=g).bfloat16()
    W = (0.05 * torch.randn(1152, 128, generator=g)).bfloat16()
    t = torch.randint(0, 1152, (600,), generator=g)
    say("lmhead grad logits pitch 1156")
    _, lse, nv, _ = _run(h, W, t)
    den = nv.to(torch.float32).clamp(min=1.0).reshape(1)
    one = torch.ones(1, device=DEV)
    a = torch.empty(600, 1152, dtype=torch.bfloat16, device=DEV)
    b = torch.empty(600, 1156, dtype=torch.bfloat16, device=DEV)
    _lib.lmhead_ce_bwd(h.to(DEV), W.to(DEV), t.to(DEV), lse, one, den, a, -100)
    _lib.lmhead_ce_bwd(h.to(DEV), W.to(DEV), t.to(DEV), lse, one, den, b, -100)
    assert torch.equal(a, b[:, :1152])


def test_lmhead_ce_grad_bad_target_rows_are_nan():
    need_gpu()
    from kernels.hip import _lib
    g = torch.Generator().manual_seed(8)
    h = torch.randn(64, 128, generator=g).bfloat16()
    W = (0.05 * torch.randn(500, 128, generator=g)).bfloat16()
    t = torch.randint(0, 500, (64,), generator=g)
    t[3] = 500
    t[5] = -100
    say("lmhead grad bad target")
    _, lse, nv, _ = _run(h, W, t)
    dz = torch.empty(64, 500, dtype=torch.bfloat16, device=DEV)
    _lib.lmhead_ce_bwd(h.to(DEV), W.to(DEV), t.to(DEV), lse, torch.ones(1, device=DEV),
                       torch.full((1,), 62.0, device=DEV), dz, -100)
    assert bool(torch.isnan(dz[3].float()).all()) and bool((dz[5].float() == 0).all())
    assert not bool(torch.isnan(dz[torch.arange(64) != 3].float()).any())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,vocab,d", [(300, 1000, 128), (1000, 4096, 256)])
def test_lmhead_ce_backward_grads(dtype, n, vocab, d):
    """grad_hidden and grad_weight of the mean loss against float64 autograd."""
    need_gpu()
    from kernels.hip.chunked_linear_cross_entropy import lmhead_ce_backward
    g = torch.Generator().manual_seed(n * 3 + vocab)
    h = torch.randn(n, d, generator=g).to(dtype)
    W = (0.05 * torch.randn(vocab, d, generator=g)).to(dtype)
    t = torch.randint(0, vocab, (n,), generator=g)
    t[::7] = -100
    say("lmhead_ce backward grads", dtype, n, vocab, d)
    loss, lse, nv, _ = _run(h, W, t)
    gh, gw = lmhead_ce_backward(h.to(DEV), W.to(DEV), t.to(DEV), lse,
                                nv.to(torch.float32).clamp(min=1.0), torch.tensor(1.3, device=DEV))
    assert gh.dtype == dtype and gw.dtype == dtype
    hr, Wr = h.double().requires_grad_(), W.double().requires_grad_()
    (1.3 * F.cross_entropy(hr @ Wr.t(), t)).backward()
    for got, want in ((gh, hr.grad), (gw, Wr.grad)):
        got = got.double().cpu()
        assert float((got - want).norm() / want.norm()) < 5e-3
        assert torch.allclose(got, want, rtol=2e-2, atol=2e-2 * float(want.abs().max()))


@pytest.mark.parametrize("softcap,ls", [(0.0, 0.0), (30.0, 0.1)])
def test_lmhead_ce_backward_vocab_ranges(monkeypatch, softcap, ls):
    """A dlogits budget below the full matrix walks the vocabulary in ranges
    (ak_lmhead_ce_bwd_range, the last one ragged): the range's dlogits equal
    the full matrix's columns bitwise, and the gradients match the one-range
    result and float64 autograd."""
    need_gpu()
    from kernels.hip import _lib
    from kernels.hip import chunked_linear_cross_entropy as clce
    g = torch.Generator().manual_seed(31)
    n, vocab, d = 700, 3000, 128
    h = torch.randn(n, d, generator=g).bfloat16()
    W = (0.05 * torch.randn(vocab, d, generator=g)).bfloat16()
    t = torch.randint(0, vocab, (n,), generator=g)
    t[::9] = -100
    t[5] = vocab - 1
    t[6] = 0
    say("lmhead_ce backward vocab ranges", softcap, ls)
    hd, Wd, td = h.to(DEV), W.to(DEV), t.to(DEV)
    _, lse, nv = clce.lmhead_ce_forward(hd, Wd, td, softcap=softcap, label_smoothing=ls)
    denom = nv.to(torch.float32).clamp(min=1.0)
    up = torch.tensor(0.7, device=DEV)
    full = torch.empty(n, vocab, dtype=torch.bfloat16, device=DEV)
    _lib.lmhead_ce_bwd(hd, Wd, td, lse, up.reshape(1), denom.reshape(1), full, -100, softcap, ls)
    for v0, v1 in ((0, 1024), (1024, 2816), (2816, 3000)):
        part = torch.empty(n, v1 - v0, dtype=torch.bfloat16, device=DEV)
        _lib.lmhead_ce_bwd_range(hd, Wd, td, lse, up.reshape(1), denom.reshape(1), part, v0, -100,
                                 softcap, ls)
        assert torch.equal(part, full[:, v0:v1]), (v0, v1)
    gh1, gw1 = clce.lmhead_ce_backward(hd, Wd, td, lse, denom, up, softcap=softcap,
                                       label_smoothing=ls)
    monkeypatch.setattr(clce, "GRAD_LOGITS_BUDGET", n * 1024 * 2)  # ranges of 1024 columns
    gh, gw = clce.lmhead_ce_backward(hd, Wd, td, lse, denom, up, softcap=softcap, label_smoothing=ls)
    # grad_weight rows: the same GEMM per row range
    assert float((gw.float() - gw1.float()).norm() / gw1.float().norm()) < 1e-3
    hr, Wr = h.double().requires_grad_(), W.double().requires_grad_()
    z = hr @ Wr.t()
    if softcap > 0:
        z = softcap * torch.tanh(z / softcap)
    (0.7 * F.cross_entropy(z, t, label_smoothing=ls)).backward()
    for got, want in ((gh, hr.grad), (gw, Wr.grad), (gh1, hr.grad)):
        got = got.double().cpu()
        assert float((got - want).norm() / want.norm()) < 5e-3


def test_c4_full_size_backward():
    """C4 backward, elementwise against the float64 oracle:
    * dlogits (the kernel's bf16) on 128 token rows x every vocab column and
      on every token x 768 vocab columns (a vocab-tile boundary, the middle
      and the ragged tail 50,176-50,303): within bf16 rounding of the oracle;
    * grad_weight on those 768 vocab rows and grad_hidden on the 128 token
      rows: tightly against the float64 GEMM of the kernel's own dlogits
      (the GEMMs' fp32 accumulation and bf16 output rounding), and against
      the oracle gradient within the bound that dlogits' bf16 rounding
      allows (2^-8 of the sum of |terms| per element);
    bf16 rounding (round to nearest, 8 significant bits) is within 2^-8 of
    the value; the bars take 1.01 times that for the fp32 arithmetic before it.
    deterministic across two calls."""
    need_gpu()
    import bench
    from kernels.hip import _lib
    from kernels.hip.chunked_linear_cross_entropy import lmhead_ce_backward
    c = bench.gen_c4()
    h, W, t = c["h"].to(DEV), c["W"].to(DEV), c["t"].to(DEV)
    say("C4 backward bf16 [8192, 768] x [50304, 768]")
    loss, lse, nv, _ = _run(c["h"], c["W"], c["t"])
    denom = nv.to(torch.float32).clamp(min=1.0)
    one = torch.ones((), device=DEV)
    gh, gw = lmhead_ce_backward(h, W, t, lse, denom, one)
    gh2, gw2 = lmhead_ce_backward(h, W, t, lse, denom, one)
    assert torch.equal(gh, gh2) and torch.equal(gw, gw2)
    dz = torch.empty(8192, 50304, dtype=torch.bfloat16, device=DEV)
    _lib.lmhead_ce_bwd(h, W, t, lse, one.reshape(1), denom.reshape(1), dz, -100)
    _, rlse, _ = _c4_oracle(c)
    tc = c["t"]
    valid = tc != -100
    scale = 1.0 / float(valid.sum())
    h64, W64 = c["h"].double(), c["W"].double()

    # vocab rows: the first tile, a tile boundary in the middle, the last tile
    # (50,176-50,303 is the ragged tail of 256-row vocab tiles) and the one before
    vsel = torch.cat([torch.arange(0, 256), torch.arange(25472, 25728), torch.arange(50048, 50304)])
    p = torch.exp(h64 @ W64[vsel].t() - rlse[:, None])             # [8192, 768]
    hit = (tc[:, None] == vsel[None, :]) & valid[:, None]
    p = (p - hit.double()) * scale
    p[~valid] = 0.0
    dzv = dz[:, vsel.to(DEV)].double().cpu()
    assert bool(((dzv - p).abs() <= _U8 * p.abs() + 1e-6 * scale).all())
    gw_sel = gw[vsel.to(DEV)].double().cpu()
    tight = dzv.t() @ h64
    terms = dzv.abs().t() @ h64.abs()
    assert bool(((gw_sel - tight).abs() <= _U8 * tight.abs() + 1e-5 * terms).all())
    ref = p.t() @ h64
    bound = (_U8 * ref.abs() + (_U8 + 2e-5) * (p.abs().t() @ h64.abs())
             + 1e-6 * scale * h64.abs().sum(0)[None, :])
    assert bool(((gw_sel - ref).abs() <= bound).all())
    del p, dzv, hit

    # token rows: 128 random rows, every vocab column
    idx = torch.randperm(8192, generator=torch.Generator().manual_seed(5))[:128].sort().values
    p = torch.exp(h64[idx] @ W64.t() - rlse[idx][:, None])           # [128, 50304]
    tv = tc[idx]
    rows = torch.arange(128)[valid[idx]]
    p[rows, tv[valid[idx]]] -= 1.0
    p *= scale
    p[~valid[idx]] = 0.0
    dzr = dz[idx.to(DEV)].double().cpu()
    assert bool(((dzr - p).abs() <= _U8 * p.abs() + 1e-6 * scale).all())
    gh_sel = gh[idx.to(DEV)].double().cpu()
    tight = dzr @ W64
    terms = dzr.abs() @ W64.abs()
    assert bool(((gh_sel - tight).abs() <= _U8 * tight.abs() + 1e-5 * terms).all())
    ref = p @ W64
    bound = (_U8 * ref.abs() + (_U8 + 2e-5) * (p.abs() @ W64.abs())
             + 1e-6 * scale * W64.abs().sum(0)[None, :])
    assert bool(((gh_sel - ref).abs() <= bound).all())


def test_c4_backward_homogeneous_in_grad_loss_bitwise():
    """Full C4: dlogits, and so both gradients, are linear in the upstream
    gradient of the loss; doubling it is exact through the dlogits epilogue,
    the GEMMs' fp32 accumulation, their partial sums and the rounding."""
    need_gpu()
    import bench
    from kernels.hip.chunked_linear_cross_entropy import lmhead_ce_backward
    c = bench.gen_c4()
    h, W, t = c["h"].to(DEV), c["W"].to(DEV), c["t"].to(DEV)
    _, lse, nv, _ = _run(c["h"], c["W"], c["t"])
    denom = nv.to(torch.float32).clamp(min=1.0)
    gh1, gw1 = lmhead_ce_backward(h, W, t, lse, denom, torch.ones((), device=DEV))
    gh2, gw2 = lmhead_ce_backward(h, W, t, lse, denom, torch.full((), 2.0, device=DEV))
    assert torch.equal(gh2, 2 * gh1) and torch.equal(gw2, 2 * gw1)


@pytest.mark.parametrize("ls", [0.0, 0.1])
def test_fused_and_row_chunked_softcap_paths_agree(ls):
    """The same softcapped (and label-smoothed) loss and gradients from the
    fused matrix-core path (bf16) and from the row-chunked GEMM + CE-kernel
    path (forced with fp32 inputs holding the same values): two independent
    implementations."""
    need_gpu()
    from kernels.hip.chunked_linear_cross_entropy import ChunkedLinearCrossEntropyLoss
    g = torch.Generator().manual_seed(12)
    h0 = torch.randn(600, 256, generator=g).bfloat16()
    W0 = (0.05 * torch.randn(5000, 256, generator=g)).bfloat16()
    t = torch.randint(0, 5000, (600,), generator=g).to(DEV)
    t[:20] = -100
    say("fused vs row-chunked softcap paths", ls)
    outs = []
    for dt in (torch.bfloat16, torch.float32):
        h = h0.to(dt).to(DEV).requires_grad_()
        W = W0.to(dt).to(DEV).requires_grad_()
        loss = ChunkedLinearCrossEntropyLoss(chunk_size=256, softcap=30.0, label_smoothing=ls,
                                             z_loss_weight=1e-4)(h, W, t)
        loss.backward()
        outs.append((float(loss), h.grad.double().cpu(), W.grad.double().cpu()))
    (l1, gh1, gw1), (l2, gh2, gw2) = outs
    assert abs(l1 - l2) <= 1e-3 * abs(l2)
    assert float((gh1 - gh2).norm() / gh2.norm()) < 1e-2
    assert float((gw1 - gw2).norm() / gw2.norm()) < 1e-2


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 100), (torch.float16, 200), (torch.bfloat16, 40),
                                     (torch.bfloat16, 256), (torch.float32, 100)])
def test_chunked_linear_ce_any_hidden_size_no_host_sync(monkeypatch, dtype, d):
    """Half-precision inputs take the matrix-core kernels at every hidden size
    (a size that is not a multiple of 64 is zero-extended; the row-chunked
    GEMM path is made to raise here), fp32 inputs the row-chunked path; the
    forward and backward of both run with torch's sync debug mode set to
    error, so neither reads a device value on the host. Loss and gradients
    against float64 autograd at the chunked-CE bars."""
    need_gpu()
    from kernels.hip import chunked_linear_cross_entropy as clce
    if dtype != torch.float32:
        def _no_fallback(*a, **k):
            raise AssertionError("half-precision input took the row-chunked GEMM path")
        monkeypatch.setattr(clce, "_chunked_forward", _no_fallback)
    g = torch.Generator().manual_seed(d)
    n, V = 333, 2100
    h0 = torch.randn(n, d, generator=g)
    W0 = 0.05 * torch.randn(V, d, generator=g)
    t = torch.randint(0, V, (n,), generator=g)
    t[::11] = -100
    say("chunked linear ce any d, no sync", dtype, d)
    h = h0.to(dtype).to(DEV).requires_grad_()
    W = W0.to(dtype).to(DEV).requires_grad_()
    td = t.to(DEV)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        loss = clce.ChunkedLinearCrossEntropyLoss(chunk_size=128, softcap=15.0)(h, W, td)
        (0.8 * loss).backward()
    finally:
        torch.cuda.set_sync_debug_mode("default")
    hr = h0.to(dtype).double().requires_grad_()
    Wr = W0.to(dtype).double().requires_grad_()
    ref = F.cross_entropy(15.0 * torch.tanh((hr @ Wr.t()) / 15.0), t)
    (0.8 * ref).backward()
    assert abs(float(loss) - float(ref)) <= 1e-3 * abs(float(ref))
    assert h.grad.shape == (n, d) and W.grad.shape == (V, d)
    for got, want in ((h.grad, hr.grad), (W.grad, Wr.grad)):
        rel = float((got.double().cpu() - want).norm() / want.norm())
        assert rel < 1e-2, rel


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_chunked_linear_ce_empty_batch(dtype):
    """No rows: loss 0 (the mean over max(1, 0) counted rows, as the
    reference's chunk loop gives), an empty hidden gradient and a zero weight
    gradient."""
    need_gpu()
    from kernels.hip.chunked_linear_cross_entropy import ChunkedLinearCrossEntropyLoss
    h = torch.zeros(0, 128, dtype=dtype, device=DEV, requires_grad=True)
    W = (0.05 * torch.randn(500, 128)).to(dtype).to(DEV).requires_grad_()
    t = torch.zeros(0, dtype=torch.int64, device=DEV)
    say("chunked linear ce empty batch", dtype)
    loss = ChunkedLinearCrossEntropyLoss()(h, W, t)
    loss.backward()
    assert float(loss) == 0.0
    assert h.grad.shape == (0, 128)
    assert W.grad is not None and bool((W.grad == 0).all())
