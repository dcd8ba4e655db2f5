"""Benchmark of the gfx950 kernel set on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only c1,c2,...] [--no-cpu]
    python bench.py --harness [KERNEL_TYPE] [--quick]

Prints ONE JSON line (the second form runs the staged correctness and timing
harness of harness.py for one kernel type and prints its report instead). The headline (``value``) is the HBM throughput of the
configuration the benchmark's metric is quoted on at one GPU: the
causal-masked fp16 row softmax [8, 12, 1024, 1024] (C2). A "step" is one
launch of that kernel over one batch of synthetic input already resident in
HBM; ``value`` = algorithmic bytes x K / wall-clock time of the K timed steps.
``roofline`` gives the kernel's achieved bandwidth from the median of at
least 100 per-launch HIP event pairs (issued while a spin kernel holds the
stream, so that they time the GPU and not the host's issue rate) against
MI355X's 8 TB/s; ``host_us_per_call`` is the host's issue time per launch;
``cpu_baseline`` times the CPU oracle on
the GPU box's host on a bounded sample of the same workload. ``kernels``
reports every configuration (C1..C5) the same way: time per launch, GB/s or
TFLOP/s, roofline fraction, tokens/s and the CPU figure beside it.

Inputs follow the seeded draw order of the survey (a CPU torch.Generator
seeded 0, then copied to the GPU). Input sets are rotated so that each timed
launch reads data not left in the 256 MB MALL by the previous launch.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "autokernel-halo-strix_amd")
if PKG not in sys.path:
    sys.path.insert(0, PKG)

import torch  # noqa: E402
import torch.nn.functional as F  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, vendor spec
BF16_PEAK_TFLOPS = 2516.6      # MI355X dense bf16 MFMA, vendor spec
ROTATE_BYTES = 640 * 2 ** 20   # > 2x the 256 MB MALL

METRIC = "HBM GB/s (% of roofline) per kernel; selective-scan Mtok/s vs CPU ref"
TRAFFIC_TABLE = os.path.join(ROOT, "profiles", "hbm_traffic_pmc.md")


def measured_traffic(kernel):
    """Calibrated HBM bytes per launch of ``kernel`` from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (None if absent)."""
    try:
        with open(TRAFFIC_TABLE) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) >= 7 and cells[0] == kernel:
                    return int(cells[4].replace(",", ""))
    except OSError:
        pass
    return None


# ---------------------------------------------------------------------------
# Synthetic inputs (seed 0, CPU generator, survey draw order)
# ---------------------------------------------------------------------------

def gen_c1():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2048, 768, generator=g)
    w = 1 + 0.02 * torch.randn(768, generator=g)
    return {"x": x, "w": w, "eps": 1e-6}


def causal_mask(n):
    return torch.triu(torch.ones(n, n, dtype=torch.bool), 1)


def gen_c2(b=8, h=12, s=1024):
    g = torch.Generator().manual_seed(0)
    x = (3 * torch.randn(b, h, s, s, generator=g)).half()
    return {"x": x.masked_fill(causal_mask(s), float("-inf"))}


def gen_c3(rows=16384, cols=4096):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(rows, cols, generator=g).bfloat16()
    r = torch.randn(rows, cols, generator=g).bfloat16()
    w = (1 + 0.02 * torch.randn(cols, generator=g)).bfloat16()
    return {"x": x, "r": r, "w": w, "eps": 1e-5}


def gen_c4(n=8192, d=768, vocab=50304, tmax=50257, ignore_frac=0.05):
    g = torch.Generator().manual_seed(0)
    h = torch.randn(n, d, generator=g).bfloat16()
    W = (0.02 * torch.randn(vocab, d, generator=g)).bfloat16()
    t = torch.randint(0, tmax, (n,), generator=g)
    t[torch.randperm(n, generator=g)[: int(ignore_frac * n)]] = -100
    return {"h": h, "W": W, "t": t}


def gen_c5(b=4, d=2048, l=4096, n=16):
    g = torch.Generator().manual_seed(0)
    u = torch.randn(b, d, l, generator=g).bfloat16()
    delta = F.softplus(0.5 * torch.randn(b, d, l, generator=g) - 4.6)
    A = -torch.arange(1, n + 1, dtype=torch.float32).expand(d, n).contiguous()
    B = torch.randn(b, 1, n, l, generator=g).bfloat16()
    C = torch.randn(b, 1, n, l, generator=g).bfloat16()
    D = torch.ones(d)
    z = torch.randn(b, d, l, generator=g).bfloat16()
    return {"u": u, "delta": delta, "A": A, "B": B, "C": C, "D": D, "z": z}


def gen_diag(b=16, l=1024, d=384):
    """Inputs of the diagonal scan as AMADEUS forms them (models/amadeus.py:98-103):
    dA = exp(dt A) with softplus-sized dt and A = -(1..64) over 6 heads,
    dBx = dt B x, C, D = 1, x ~ N(0, 1), and an upstream gradient."""
    g = torch.Generator().manual_seed(3)
    dt = F.softplus(torch.randn(b, l, d, generator=g) * 0.5 - 4.0)
    A = -torch.arange(1, 65, dtype=torch.float32).repeat(d // 64)
    x = torch.randn(b, l, d, generator=g)
    return {"dA": torch.exp(dt * A), "dBx": dt * torch.randn(b, l, d, generator=g) * x,
            "C": torch.randn(b, l, d, generator=g), "D": torch.ones(d), "x": x,
            "gy": torch.randn(b, l, d, generator=g)}


# Algorithmic work per launch (survey 8(d)).
C1_BYTES = 2048 * 768 * 4 * 2 + 768 * 4
C2_BYTES = 2 * 8 * 12 * 1024 * 1024 * 2
C3_BYTES = 4 * 16384 * 4096 * 2 + 4096 * 2
# fused residual + RMSNorm backward at the C3 shape: read hidden, grad_hidden,
# grad_normed, weight; write grad_x and the fp32 weight gradient
C3B_BYTES = 4 * 16384 * 4096 * 2 + 4096 * 2 + 4096 * 4
C4_FLOP = 2 * 8192 * 50304 * 768
C4_MIN_BYTES = 8192 * 768 * 2 + 50304 * 768 * 2 + 8192 * 8 + 8192 * 4 + 4
# backward: logits recomputed on the matrix cores, then grad_hidden and
# grad_weight GEMMs: three products of 2 N V D flop each
C4B_FLOP = 3 * C4_FLOP
C5_BYTES = 3 * 4 * 2048 * 4096 * 2 + 4 * 2048 * 4096 * 4 + 2 * 4 * 16 * 4096 * 2 + 2048 * 16 * 4 + 2048 * 4
# the reference's N=64 mamba-ssm shape: u, delta, out fp16 [8, 384, 512];
# B, C fp16 [8, 64, 512]; A [384, 64] and D fp32
N64_BYTES = 3 * 8 * 384 * 512 * 2 + 2 * 8 * 64 * 512 * 2 + 384 * 64 * 4 + 384 * 4
# the diagonal scan (AMADEUS's SSM path, 384 channels) at batch 16, seqlen 1024:
# forward reads dA, dBx, C, x and writes y (fp32 per element) plus D; backward
# reads dA, dBx, C, x, grad_y and writes grad_dA, grad_dBx, grad_C, grad_x,
# plus D and grad_D
DIAG_SHAPE = (16, 1024, 384)
DIAG_BYTES = 5 * 4 * 16 * 1024 * 384 + 384 * 4
DIAGB_BYTES = 9 * 4 * 16 * 1024 * 384 + 2 * 384 * 4
# Mamba-1 backward at the C5 shape: read u, z, dout (bf16), delta (fp32), B, C,
# A, D; write du, dz (bf16), ddelta (fp32), dB, dC (bf16), dA, dD (fp32)
C5B_BYTES = (4 * 2048 * 4096 * (2 + 2 + 2 + 4 + 2 + 2 + 4) + 4 * 4 * 16 * 4096 * 2
             + 2 * (2048 * 16 * 4 + 2048 * 4))


# ---------------------------------------------------------------------------
# GPU side: the product's C-ABI launchers with preallocated outputs
# ---------------------------------------------------------------------------

def _sets(nbytes):
    return max(1, min(64, math.ceil(ROTATE_BYTES / max(1, nbytes))))


def _replicate(tensors, k):
    """k device copies of a dict of CPU tensors (first copy shares nothing with the CPU)."""
    out = []
    for _ in range(k):
        out.append({n: (v.cuda() if torch.is_tensor(v) else v) for n, v in tensors.items()})
    return out


class Case:
    """One configuration: device state, one launch per step, algorithmic work."""

    def __init__(self, name, workload, bound, work, unit_tokens, launch, sets, kernel_name,
                 valu_cycles=None, valu_model=None):
        self.name, self.workload, self.bound, self.work = name, workload, bound, work
        self.tokens, self.launch, self.sets, self.kernel_name = unit_tokens, launch, sets, kernel_name
        # VALU issue cycles of the whole launch (wave64 instructions x their
        # issue cost per SIMD), for kernels whose floor is instruction issue
        self.valu_cycles, self.valu_model = valu_cycles, valu_model


# gfx950 issue cost per wave64 instruction and SIMD, measured with a
# throughput probe on the box (8 independent chains per lane, 8 waves per SIMD)
CYC_DPP_MUL, CYC_EXP, CYC_FMA = 4.7, 9.8, 3.0
# The scan's work per (step, state) and lane: 2 DPP-broadcast multiplies
# (decay exponent, delta u B), 1 exp2, the state FMA and the output FMA.
SCAN_CYC_PER_STATE_STEP = 2 * CYC_DPP_MUL + CYC_EXP + 2 * CYC_FMA
SCAN_VALU_MODEL = ("per (step, state) and wave64: 2 v_mul_f32_dpp (4.7 cyc) + v_exp_f32 (9.8) "
                   "+ 2 v_fmac_f32 (3.0), 64 (channel, state) lanes per wave, 1024 SIMDs at 2.4 GHz")


def scan_valu_cycles(batch, dim, dstate, seqlen):
    waves = batch * dim * max(16, dstate) / 64
    return waves * seqlen * SCAN_CYC_PER_STATE_STEP


def make_case(name):
    from kernels.hip import _lib
    if name == "c1":
        cpu = gen_c1()
        k = _sets(C1_BYTES)
        sets = _replicate(cpu, k)
        for s in sets:
            s["y"] = torch.empty_like(s["x"])
        # the lean launcher kernels.hip.rmsnorm.kernel_fn uses for contiguous
        # rows (dense pitch, no 2-D views): a 5 us kernel is issue-bound
        launch = lambda s: _lib.rmsnorm_contig(s["x"], s["w"], s["y"], 768, s["eps"])
        return Case(name, "C1 RMSNorm fp32 [2048, 768]", "hbm", C1_BYTES, 2048, launch, sets,
                    "rownorm_vec_kernel")
    if name == "c2":
        cpu = gen_c2()
        k = _sets(C2_BYTES)
        sets = _replicate(cpu, k)
        for s in sets:
            s["x2"] = s["x"].view(-1, 1024)
            s["y"] = torch.empty_like(s["x2"])
        launch = lambda s: _lib.softmax(s["x2"], s["y"])
        return Case(name, "C2 causal softmax fp16 [8, 12, 1024, 1024]", "hbm", C2_BYTES, 98304,
                    launch, sets, "softmax_vec_kernel")
    if name == "c3":
        cpu = gen_c3()
        k = _sets(C3_BYTES)
        sets = _replicate(cpu, k)
        for s in sets:
            s["nr"] = torch.empty_like(s["x"])
            s["y"] = torch.empty_like(s["x"])
        launch = lambda s: _lib.fused_add_rmsnorm(s["x"], s["r"], s["w"], s["nr"], s["y"], s["eps"])
        return Case(name, "C3 fused residual + RMSNorm bf16 [16384, 4096]", "hbm", C3_BYTES, 16384,
                    launch, sets, "rownorm_vec_kernel")
    if name == "c3b":
        c = gen_c3()
        g = torch.Generator().manual_seed(1)
        cpu = {"h": (c["x"] + c["r"]), "w": c["w"],
               "gh": torch.randn(16384, 4096, generator=g).bfloat16(),
               "gn": torch.randn(16384, 4096, generator=g).bfloat16(), "eps": c["eps"]}
        k = _sets(C3B_BYTES)
        sets = _replicate(cpu, k)
        wsb = _lib.rmsnorm_bwd_workspace_bytes(16384, 4096)
        for s in sets:
            s["gx"] = torch.empty_like(s["h"])
            s["gw"] = torch.empty(4096, dtype=torch.float32, device="cuda")
            s["ws"] = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        launch = lambda s: _lib.fused_add_rmsnorm_bwd(s["h"], s["w"], s["gh"], s["gn"], s["gx"],
                                                      s["gw"], s["ws"], s["eps"])
        return Case(name, "C3-shape fused residual + RMSNorm backward bf16 [16384, 4096]", "hbm",
                    C3B_BYTES, 16384, launch, sets, "rownorm_bwd_vec_kernel")
    if name == "c4":
        cpu = gen_c4()
        sets = _replicate(cpu, 2)
        wsb = _lib.lmhead_ce_workspace_bytes(8192, 50304)
        for s in sets:
            s["loss"] = torch.empty((), dtype=torch.float32, device="cuda")
            s["lse"] = torch.empty(8192, dtype=torch.float32, device="cuda")
            s["nv"] = torch.empty(1, dtype=torch.int64, device="cuda")
            s["ws"] = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        launch = lambda s: _lib.lmhead_ce(s["h"], s["W"], s["t"], s["loss"], s["lse"], None, s["nv"],
                                          s["ws"], -100)
        return Case(name, "C4 lm-head + CE bf16 [8192, 768] x [50304, 768]", "mfma", C4_FLOP, 8192,
                    launch, sets, "lmhead_ce_tile_kernel")
    if name == "c4s":
        cpu = gen_c4()
        sets = _replicate(cpu, 2)
        wsb = _lib.lmhead_ce_workspace_bytes(8192, 50304)
        for s in sets:
            s["loss"] = torch.empty((), dtype=torch.float32, device="cuda")
            s["lse"] = torch.empty(8192, dtype=torch.float32, device="cuda")
            s["nv"] = torch.empty(1, dtype=torch.int64, device="cuda")
            s["ws"] = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        launch = lambda s: _lib.lmhead_ce(s["h"], s["W"], s["t"], s["loss"], s["lse"], None, s["nv"],
                                          s["ws"], -100, 30.0)
        return Case(name, "C4 lm-head + CE bf16 with logit softcap 30 (the reference's usual setting)",
                    "mfma", C4_FLOP, 8192, launch, sets, "lmhead_ce_tile_kernel (softcap)")
    if name == "c4b":
        from kernels.hip.chunked_linear_cross_entropy import lmhead_ce_backward, lmhead_ce_forward
        cpu = gen_c4()
        sets = _replicate(cpu, 2)
        for s in sets:
            _, s["lse"], nv = lmhead_ce_forward(s["h"], s["W"], s["t"])
            s["den"] = nv.to(torch.float32).clamp(min=1.0)
            s["g"] = torch.ones((), dtype=torch.float32, device="cuda")
        launch = lambda s: lmhead_ce_backward(s["h"], s["W"], s["t"], s["lse"], s["den"], s["g"])
        return Case(name, "C4 lm-head + CE backward bf16 (dlogits on the matrix cores + 2 GEMMs)",
                    "mfma", C4B_FLOP, 8192, launch, sets, "lmhead_ce_tile_kernel (grad) + GEMMs")
    if name == "c5":
        cpu = gen_c5()
        k = _sets(C5_BYTES)
        sets = _replicate(cpu, k)
        for s in sets:
            s["out"] = torch.empty_like(s["u"])
        launch = lambda s: _lib.selective_scan(s["u"], s["delta"], s["A"], s["B"], s["C"], s["D"],
                                               s["z"], None, s["out"], None, False)
        return Case(name, "C5 Mamba-1 selective scan B4 L4096 D2048 N16", "hbm", C5_BYTES, 4 * 4096,
                    launch, sets, "mamba_scan_split_kernel (producer / consumer waves)",
                    valu_cycles=scan_valu_cycles(4, 2048, 16, 4096), valu_model=SCAN_VALU_MODEL)
    if name == "n64":
        # the reference's own mamba-ssm benchmark shape (scripts/bench_external_kernels.py:140)
        g = torch.Generator().manual_seed(0)
        cpu = {"u": torch.randn(8, 384, 512, generator=g).half(),
               "delta": torch.randn(8, 384, 512, generator=g).half(),
               "A": -torch.rand(384, 64, generator=g),
               "B": torch.randn(8, 1, 64, 512, generator=g).half(),
               "C": torch.randn(8, 1, 64, 512, generator=g).half(),
               "D": torch.randn(384, generator=g)}
        sets = _replicate(cpu, _sets(N64_BYTES))
        for s in sets:
            s["out"] = torch.empty_like(s["u"])
        launch = lambda s: _lib.selective_scan(s["u"], s["delta"], s["A"], s["B"], s["C"], s["D"],
                                               None, None, s["out"], None, True)
        return Case(name, "Mamba-1 scan at the reference's benchmark shape B8 D384 L512 N64 fp16",
                    "hbm", N64_BYTES, 8 * 512, launch, sets, "mamba_scan_fast_kernel (4 lane rows per channel)",
                    valu_cycles=scan_valu_cycles(8, 384, 64, 512), valu_model=SCAN_VALU_MODEL)
    if name in ("diag", "diagb"):
        # the diagonal recurrence at AMADEUS's shape: chunked forward / backward
        cpu = gen_diag(*DIAG_SHAPE)
        sets = _replicate(cpu, _sets(DIAGB_BYTES if name == "diagb" else DIAG_BYTES))
        for st in sets:
            st["y"] = torch.empty_like(st["x"])
            st["grads"] = [torch.empty_like(st["x"]) for _ in range(4)] + [torch.empty_like(st["D"])]
        if name == "diag":
            launch = lambda st: _lib.diag_scan(st["dA"], st["dBx"], st["C"], st["D"], st["x"], st["y"])
            return Case(name, "Diagonal scan fp32 [16, 1024, 384] (AMADEUS's SSM width)", "hbm", DIAG_BYTES,
                        16 * 1024, launch, sets,
                        "diag_scan_wg_kernel (one launch, 32 channels per workgroup)")
        launch = lambda st: _lib.diag_scan_bwd(st["dA"], st["dBx"], st["C"], st["D"], st["x"], st["gy"],
                                               st["grads"][0], st["grads"][1], st["grads"][2], st["grads"][4],
                                               st["grads"][3])
        return Case(name, "Diagonal scan backward fp32 [16, 1024, 384]", "hbm", DIAGB_BYTES, 16 * 1024, launch,
                    sets, "diag_bwd_wg_carry_kernel + diag_bwd_chunk_kernel<32> + diag_scan_gd_kernel")
    if name == "c5b":
        cpu = gen_c5()
        cpu["dout"] = torch.randn(cpu["u"].shape, generator=torch.Generator().manual_seed(2)).bfloat16()
        sets = _replicate(cpu, 2)
        for s in sets:
            for k in ("du", "dz"):
                s[k] = torch.empty_like(s["u"])
            s["ddelta"] = torch.empty_like(s["delta"])
            s["dA"] = torch.empty_like(s["A"])
            s["dB"] = torch.empty_like(s["B"])
            s["dC"] = torch.empty_like(s["C"])
            s["dD"] = torch.empty_like(s["D"])
        launch = lambda s: _lib.selective_scan_bwd(
            s["u"], s["delta"], s["A"], s["B"], s["C"], s["D"], s["z"], None, s["dout"], s["du"],
            s["ddelta"], s["dA"], s["dB"], s["dC"], s["dD"], s["dz"], None, False)
        return Case(name, "C5-shape Mamba-1 selective scan backward B4 L4096 D2048 N16", "hbm",
                    C5B_BYTES, 4 * 4096, launch, sets,
                    "mamba_scan_split_kernel (preparation) + mamba_scan_bwd_fast_kernel + scan_bwd_bc_sum4_kernel (with the per-batch sums)")
    if name == "c5t":
        # one training step of the scan: the forward keeps its states every 16
        # steps and its pre-gate output, the backward restarts from them
        cpu = gen_c5()
        cpu["dout"] = torch.randn(cpu["u"].shape, generator=torch.Generator().manual_seed(2)).bfloat16()
        sets = _replicate(cpu, 2)
        for s in sets:
            for k in ("out", "prez", "du", "dz"):
                s[k] = torch.empty_like(s["u"])
            s["ck"] = torch.empty((4, 4096 // 16, 2048, 16), dtype=torch.float32, device="cuda")
            s["ddelta"] = torch.empty_like(s["delta"])
            s["dA"] = torch.empty_like(s["A"])
            s["dB"] = torch.empty_like(s["B"])
            s["dC"] = torch.empty_like(s["C"])
            s["dD"] = torch.empty_like(s["D"])

        def launch(s):
            _lib.selective_scan(s["u"], s["delta"], s["A"], s["B"], s["C"], s["D"], s["z"], None,
                                s["out"], None, False, out_prez=s["prez"], checkpoints=s["ck"])
            _lib.selective_scan_bwd(s["u"], s["delta"], s["A"], s["B"], s["C"], s["D"], s["z"], None,
                                    s["dout"], s["du"], s["ddelta"], s["dA"], s["dB"], s["dC"], s["dD"],
                                    s["dz"], None, False, checkpoints=s["ck"], out_prez=s["prez"])
        return Case(name, "C5-shape Mamba-1 training step (forward keeping its states + backward from them)",
                    "hbm", C5_BYTES + C5B_BYTES, 4 * 4096, launch, sets,
                    "mamba_scan_split_kernel (training variant) + mamba_scan_bwd_fast_kernel + scan_bwd_bc_sum4_kernel (with the per-batch sums)")
    raise ValueError(name)


# Launches timed one by one (an event pair each) for the roofline figures,
# whatever --steps is.
ROOFLINE_PAIRS = 100


def time_case(case, steps, warmup, pairs=ROOFLINE_PAIRS):
    """W untimed steps, then K timed steps bracketed by synchronisations.

    Returns (wall seconds of the K steps, mean ms per launch from one HIP
    event pair around the K back-to-back launches on the launch stream,
    median ms per launch over ``pairs`` (>= 100) launches each bracketed by
    its own event pair and queued behind a held stream, host us per
    launcher call, mean ms per launch over about SUSTAIN_S seconds of
    back-to-back launches, and that run's launch count)."""
    nset = len(case.sets)
    for i in range(warmup):
        case.launch(case.sets[i % nset])
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for i in range(steps):
        case.launch(case.sets[i % nset])
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    mean_ms = ev0.elapsed_time(ev1) / steps
    n = max(pairs, ROOFLINE_PAIRS)
    durations, host_us = held_event_pairs(case, n)
    med_ms = statistics.median(durations)
    sus_ms, sus_n = sustained_run(case, med_ms)
    return wall, mean_ms, med_ms, host_us, sus_ms, sus_n


# Seconds of back-to-back launches behind the sustained figure (at least 20
# and at most 5000 launches). A kernel launched after an idle or lighter
# phase runs its first few milliseconds in a power-management transient
# (the clock overshoots, then throttles back); a run this long reports the
# rate the kernel settles at.
SUSTAIN_S = 0.25


def sustained_run(case, med_ms):
    """Mean ms per launch over about SUSTAIN_S seconds of back-to-back
    launches (one event pair around them), and the launch count."""
    nset = len(case.sets)
    n = int(min(5000, max(20, SUSTAIN_S / (med_ms * 1e-3))))
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for i in range(n):
        case.launch(case.sets[i % nset])
    ev1.record()
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / n, n


# GPU cycles of the spin kernel that holds the stream before each batch of
# event pairs (about 1 ms at MI355X clocks); doubled when a batch drained.
HOLD_CYCLES = 2_000_000
PAIR_BATCH = 25


def held_event_pairs(case, n):
    """Per-launch GPU durations (ms) from ``n`` event pairs, and the host time
    per launcher call (us).

    A launch of a few microseconds takes less GPU time than the host needs to
    issue it and its two event records, so pairs issued back to back would
    time the host's issue rate, not the kernel. Each batch of pairs is
    therefore queued behind a spin kernel (``torch.cuda._sleep``): the host
    issues the whole batch while the GPU spins, and the GPU then runs the
    pairs back to back. A batch whose last event has already completed when
    the host finishes issuing it may hold host gaps; it is issued again with a
    longer spin. The host time per call is the issue time of a batch of
    launches without event records, also behind a held stream, over its
    launches (median of four batches)."""
    nset = len(case.sets)
    durations, host = [], []
    hold = HOLD_CYCLES
    i = 0
    while i < n:
        b = min(PAIR_BATCH, n - i)
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(b)]
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(b)]
        torch.cuda._sleep(hold)
        for j in range(b):
            starts[j].record()
            case.launch(case.sets[(i + j) % nset])
            ends[j].record()
        drained = ends[-1].query()
        torch.cuda.synchronize()
        if drained and hold < 64 * HOLD_CYCLES:
            hold *= 2
            continue
        durations += [s.elapsed_time(e) for s, e in zip(starts, ends)]
        i += b
    for _ in range(4):
        torch.cuda._sleep(hold)
        t0 = time.perf_counter()
        for j in range(PAIR_BATCH):
            case.launch(case.sets[j % nset])
        host.append((time.perf_counter() - t0) / PAIR_BATCH * 1e6)
        torch.cuda.synchronize()
    return durations, statistics.median(host)


# ---------------------------------------------------------------------------
# CPU baseline: the oracle on a bounded sample, on the host's cores
# ---------------------------------------------------------------------------

def cpu_baseline(name, budget_s=4.0):
    """Returns (rate, unit, sample description) for the CPU oracle on a sample of ``name``."""
    from oracle import ops

    def timed(fn, reps, budget=None):
        fn()
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t)
            if sum(ts) > (budget or budget_s):
                break
        return statistics.median(ts)

    if name == "c1":
        c = gen_c1()
        t = timed(lambda: ops.rmsnorm_ref(c["x"], c["w"], c["eps"]), 5)
        return C1_BYTES / t / 1e9, "GB/s", "full C1 (2048 x 768 fp32)"
    if name == "c2":
        # the headline's baseline: the whole C2 workload, repeated for about
        # 10 s of CPU work (median of the repetitions)
        c = gen_c2()
        t = timed(lambda: ops.softmax_ref(c["x"]), 1000, budget=10.0)
        return C2_BYTES / t / 1e9, "GB/s", "full C2 (96 planes), repeated for about 10 s, median"
    if name == "c3":
        c = gen_c3(rows=1024)
        t = timed(lambda: ops.fused_residual_add_rmsnorm_ref(c["x"], c["r"], c["w"], c["eps"]), 5)
        return C3_BYTES * (1024 / 16384) / t / 1e9, "GB/s", "1024 of 16384 rows of C3"
    if name == "c3b":
        c = gen_c3(rows=1024)
        g = torch.Generator().manual_seed(1)
        h = c["x"] + c["r"]
        gh = torch.randn(1024, 4096, generator=g).bfloat16()
        gn = torch.randn(1024, 4096, generator=g).bfloat16()
        t = timed(lambda: ops.fused_residual_rmsnorm_bwd_ref(h, c["w"], gh, gn, c["eps"]), 5)
        return C3B_BYTES * (1024 / 16384) / t / 1e9, "GB/s", "1024 of 16384 rows of the C3-shape backward (float64 oracle)"
    if name == "c4":
        c = gen_c4()
        rows = 64
        h, t_ = c["h"][:rows], c["t"][:rows]
        t = timed(lambda: ops.lmhead_ce_ref(h, c["W"], t_), 3)
        return 2 * rows * 50304 * 768 / t / 1e12, "TFLOP/s", f"{rows} of 8192 rows of C4 (fp32 GEMM per 4096-column vocab chunk)"
    if name == "c4s":
        c = gen_c4()
        rows = 64
        h, t_ = c["h"][:rows], c["t"][:rows]
        t = timed(lambda: ops.lmhead_ce_ref(h, c["W"], t_, softcap=30.0), 3)
        return 2 * rows * 50304 * 768 / t / 1e12, "TFLOP/s", f"{rows} of 8192 rows of C4 with softcap 30 (fp32 GEMM per 4096-column vocab chunk)"
    if name == "c4b":
        c = gen_c4()
        rows = 32
        h, t_ = c["h"][:rows].float(), c["t"][:rows]
        Wf = c["W"].float()

        def bwd():
            z = h @ Wf.t()
            p = torch.softmax(z, -1)
            p[torch.arange(rows), t_.clamp(min=0)] -= 1.0
            p[t_ == -100] = 0.0
            return p @ Wf, p.t() @ h
        t = timed(bwd, 3)
        return 3 * 2 * rows * 50304 * 768 / t / 1e12, "TFLOP/s", f"{rows} of 8192 rows of the C4 backward (fp32 torch)"
    if name == "c5":
        c = gen_c5(b=1, d=64)
        t = timed(lambda: ops.selective_scan_ref(c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"],
                                                 c["z"]), 1)
        # tokens/s of the full problem = (channel-steps/s) / dim
        return (64 * 4096) / t / 2048 / 1e6, "Mtok/s", "batch 1, 64 of 2048 channels, full L=4096"
    if name == "c5b":
        c = gen_c5(b=1, d=32)
        dout = torch.randn(c["u"].shape, generator=torch.Generator().manual_seed(2)).bfloat16()
        t = timed(lambda: ops.selective_scan_bwd_ref(c["u"], c["delta"], c["A"], c["B"], c["C"], dout,
                                                     c["D"], c["z"]), 2)
        return (32 * 4096) / t / 2048 / 1e6, "Mtok/s", "batch 1, 32 of 2048 channels, full L=4096 (float64 oracle)"
    if name == "c5t":
        c = gen_c5(b=1, d=32)
        dout = torch.randn(c["u"].shape, generator=torch.Generator().manual_seed(2)).bfloat16()
        t = timed(lambda: (ops.selective_scan_ref(c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["z"]),
                           ops.selective_scan_bwd_ref(c["u"], c["delta"], c["A"], c["B"], c["C"], dout,
                                                      c["D"], c["z"])), 2)
        return ((32 * 4096) / t / 2048 / 1e6, "Mtok/s",
                "batch 1, 32 of 2048 channels, full L=4096 (forward oracle + float64 backward oracle)")
    if name == "diag":
        c = gen_diag(b=1)
        t = timed(lambda: ops.diag_scan_ref(c["dA"], c["dBx"], c["C"], c["D"], c["x"]), 3)
        return DIAG_BYTES / 16 / t / 1e9, "GB/s", "batch 1 of 16 (fp32 oracle)"
    if name == "diagb":
        c = gen_diag(b=1)
        t = timed(lambda: ops.diag_scan_bwd_ref(c["dA"], c["dBx"], c["C"], c["D"], c["x"], c["gy"]), 2)
        return DIAGB_BYTES / 16 / t / 1e9, "GB/s", "batch 1 of 16 (float64 oracle)"
    if name == "n64":
        g = torch.Generator().manual_seed(0)
        u = torch.randn(1, 48, 512, generator=g).half()
        delta = torch.randn(1, 48, 512, generator=g).half()
        A = -torch.rand(48, 64, generator=g)
        B = torch.randn(1, 64, 512, generator=g).half()
        C = torch.randn(1, 64, 512, generator=g).half()
        D = torch.randn(48, generator=g)
        t = timed(lambda: ops.selective_scan_ref(u, delta, A, B, C, D, None, None, True), 3)
        return (48 * 512) / t / 384 / 1e6, "Mtok/s", "batch 1, 48 of 384 channels, full L=512"
    raise ValueError(name)


# ---------------------------------------------------------------------------

def cpu_model() -> str:
    """The host CPU's model name (from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default="c1,c2,c3,c3b,c4,c4s,c4b,c5,c5b,c5t,n64,diag,diagb")
    ap.add_argument("--harness", nargs="?", const="", default=None, metavar="KERNEL_TYPE",
                    help="run the staged correctness + timing harness for one kernel type "
                         "(softmax, cross_entropy, rmsnorm, fused_residual_add_rmsnorm, "
                         "selective_scan; default: kernel.py's) instead of the JSON benchmark")
    ap.add_argument("--quick", action="store_true", help="harness: skip stages 3-5")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run 3 device copies of 256 MiB (a known-size kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args(argv)
    if args.harness is not None:
        if not torch.cuda.is_available():
            print("the harness needs a GPU", file=sys.stderr)
            return 2
        import harness
        hargs = (["--kernel", args.harness] if args.harness else []) + (["--quick"] if args.quick else [])
        out = harness.main(hargs)
        return 0 if out["correctness"]["correctness"] == "PASS" else 1
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)
    if args.copy_calibration:
        src = torch.ones(256 * 2 ** 20 // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    names = [n.strip() for n in args.only.split(",") if n.strip()]
    if "c2" not in names:
        names.insert(0, "c2")
    kernels = {}
    head = None
    for name in names:
        case = make_case(name)
        wall, mean_ms, med_ms, host_us, sus_ms, sus_n = time_case(case, args.steps, args.warmup, args.steps)
        # rooflines from the median of the per-launch event pairs
        if case.bound == "hbm":
            achieved = case.work / (med_ms * 1e-3) / 1e9
            peak, unit = HBM_PEAK_GBS, "GB/s"
        else:
            achieved = case.work / (med_ms * 1e-3) / 1e12
            peak, unit = BF16_PEAK_TFLOPS, "TFLOP/s"
        sustained = achieved * med_ms / sus_ms
        rec = {
            "workload": case.workload,
            "kernel": case.kernel_name,
            "us_per_launch_median_event_pairs": round(med_ms * 1e3, 2),
            "event_pairs": max(ROOFLINE_PAIRS, args.steps),
            "achieved": round(achieved, 1),
            "unit": unit,
            "peak": peak,
            "frac": round(achieved / peak, 4),
            # the K timed back-to-back launches (one event pair around them),
            # which start in the power-management transient
            "us_per_launch_mean": round(mean_ms * 1e3, 2),
            "frac_mean": round(achieved * med_ms / mean_ms / peak, 4),
            # about SUSTAIN_S seconds of back-to-back launches: the settled rate
            "us_per_launch_sustained": round(sus_ms * 1e3, 2),
            "sustained_launches": sus_n,
            "achieved_sustained": round(sustained, 1),
            "frac_sustained": round(sustained / peak, 4),
            "tokens_per_s": round(case.tokens / (med_ms * 1e-3), 1),
            "input_sets": len(case.sets),
            "wall_ms_per_step": round(wall / args.steps * 1e3, 4),
            "host_us_per_call": round(host_us, 2),
        }
        if case.valu_cycles:
            # the VALU issue floor: instruction cycles per wave64 and SIMD over
            # MI355X's 1024 SIMDs at the 2.4 GHz peak clock
            floor_us = case.valu_cycles / 1024 / 2.4e3
            rec["valu_roofline"] = {"floor_us": round(floor_us, 1),
                                    "frac": round(floor_us / (med_ms * 1e3), 4),
                                    "frac_sustained": round(floor_us / (sus_ms * 1e3), 4),
                                    "model": case.valu_model}
        if name.startswith("c5") or name == "n64":
            rec["Mtok_per_s"] = round(case.tokens / (med_ms * 1e-3) / 1e6, 2)
        if not args.no_cpu:
            rate, cunit, sample = cpu_baseline(name)
            rec["cpu"] = {"value": round(rate, 4), "unit": cunit, "sample": sample}
            gpu_same_unit = rec.get("Mtok_per_s") if cunit == "Mtok/s" else achieved
            rec["gpu_over_cpu"] = round(gpu_same_unit / rate, 1) if rate > 0 else None
        kernels[name] = rec
        if name == "c2":
            head = (case, wall, mean_ms)
        del case
        torch.cuda.empty_cache()

    case, wall, mean_ms = head
    value = C2_BYTES * args.steps / wall / 1e9
    h = kernels["c2"]
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seed-0 CPU generator, survey draw order)",
        "config": {"workload": case.workload, "rows": 98304, "cols": 1024, "mask": "causal -inf",
                   "accumulate": "fp32", "input_sets_rotated": len(case.sets)},
        "roofline": {"bound": "hbm", "achieved": h["achieved"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": h["frac"], "traffic": measured_traffic("softmax_vec_kernel"),
                     "achieved_from": f"median of {h['event_pairs']} per-launch HIP event pairs, "
                                      "issued in batches queued behind a held stream",
                     "traffic_from": "profiles/hbm_traffic_pmc.md: rocprofv3 FETCH_SIZE + WRITE_SIZE "
                                     "per dispatch, scaled by a 256 MiB copy's readings"},
        "cpu_baseline": None,
        "kernels": kernels,
        "host": {"cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
                 "cpu": cpu_model(), "torch": torch.__version__,
                 "gpu": torch.cuda.get_device_name(0),
                 "gpu_arch": getattr(torch.cuda.get_device_properties(0), "gcnArchName", "unknown"),
                 "gpu_cus": torch.cuda.get_device_properties(0).multi_processor_count},
    }
    if "cpu" in h:
        line["cpu_baseline"] = {"value": h["cpu"]["value"], "unit": "GB/s",
                                "cores": torch.get_num_threads(), "kind": "port",
                                "sample": h["cpu"]["sample"]}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
