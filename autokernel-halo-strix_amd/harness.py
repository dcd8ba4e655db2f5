"""Kernel harness: staged correctness checks and timing for one kernel type.

The gfx950 counterpart of the reference's ``bench.py`` harness
(``KERNEL_CONFIGS`` :459-752, ``run_correctness`` :1038-1363, the timing of
:1370-1500 and the greppable summary :1796-1806). ``python bench.py
--harness rmsnorm`` (or ``python -m harness --kernel rmsnorm`` from the
package directory) runs it and prints the reference's report, ending in::

    === FINAL ===
    kernel_type: rmsnorm
    correctness: PASS
    throughput_tflops: ...
    speedup_vs_pytorch: ...x
    pct_peak_compute: ...%
    bench_time_seconds: ...

Kernel types: ``softmax``, ``cross_entropy``, ``rmsnorm``,
``fused_residual_add_rmsnorm`` (the north star's kernel set with a
materialised-logits CE) and ``selective_scan`` (Mamba-1). Sizes are the
reference's own plus the MI355X configurations the library is measured on
(``c1``..``c5``).

Correctness runs five stages, as the reference does: a smoke test on the
first size, a sweep over every size and dtype, the five adversarial input
transforms (near_max, near_zero, mixed_scale, all_zeros, all_same), three
runs that must agree bit for bit, and sizes off the power-of-two grid. Each
kernel is checked against eager PyTorch evaluating the reference's formula
(``reference.py``) in fp32 and rounding once -- the parity bar the kernels
are built to -- at the reference harness's tolerances. Timing takes the
median of at least 100 launches, each bracketed by its own HIP event pair on
the launching stream, for the kernel and for the same eager PyTorch formula
("speedup_vs_pytorch"); rooflines use MI355X peaks (8 TB/s HBM3E, 2516.6
TFLOP/s dense bf16 / fp16).
"""

from __future__ import annotations

import argparse
import math
import sys
import time
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

PEAK_HBM_GBS = 8000.0
PEAK_TFLOPS_16 = 2516.6

Size = Dict[str, int]


@dataclass
class KernelSpec:
    """One kernel type: its sizes, dtypes, tolerances, inputs, reference and
    kernel (the fields of a reference ``KERNEL_CONFIGS`` entry)."""
    kernel_type: str
    test_sizes: List[Tuple[str, Size]]
    test_dtypes: List[torch.dtype]
    tolerances: Dict[torch.dtype, Dict[str, float]]
    input_generator: Callable[[Size, torch.dtype, str, int], dict]
    reference_fn: Callable[[dict], torch.Tensor]
    kernel_fn: Callable[..., torch.Tensor]
    flops_fn: Callable[[Size], int]
    bytes_fn: Callable[[Size, torch.dtype], int]
    edge_sizes: List[Tuple[str, Size]] = field(default_factory=list)
    primary: str = "large"
    adversarial: bool = True   # run stage 3's input transforms


def _esize(dt: torch.dtype) -> int:
    return torch.tensor([], dtype=dt).element_size()


def _gen(seed: int, device: str) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(seed)


# ---------------------------------------------------------------------------
# Inputs (drawn on the device from a seeded generator) and references
# ---------------------------------------------------------------------------

def _softmax_inputs(s, dt, dev, seed):
    return {"x": torch.randn(s["rows"], s["cols"], device=dev, generator=_gen(seed, dev)).to(dt)}


def _softmax_ref(i):
    return torch.softmax(i["x"].float(), dim=-1).to(i["x"].dtype)


def _ce_inputs(s, dt, dev, seed):
    g = _gen(seed, dev)
    logits = torch.randn(s["batch"], s["vocab"], device=dev, generator=g).to(dt)
    targets = torch.randint(0, s["vocab"], (s["batch"],), device=dev, generator=g)
    return {"logits": logits, "targets": targets}


def _ce_ref(i):
    return F.cross_entropy(i["logits"].float(), i["targets"])


def _rms_inputs(s, dt, dev, seed):
    g = _gen(seed, dev)
    return {"x": torch.randn(s["M"], s["N"], device=dev, generator=g).to(dt),
            "weight": torch.randn(s["N"], device=dev, generator=g).to(dt)}


def _rms_ref(i):
    x = i["x"].float()
    rms = torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6)
    return ((x / rms) * i["weight"].float()).to(i["x"].dtype)


def _fused_inputs(s, dt, dev, seed):
    g = _gen(seed, dev)
    return {"x": torch.randn(s["M"], s["N"], device=dev, generator=g).to(dt),
            "residual": torch.randn(s["M"], s["N"], device=dev, generator=g).to(dt),
            "weight": torch.randn(s["N"], device=dev, generator=g).to(dt)}


def _fused_ref(i):
    h = (i["x"] + i["residual"]).float()
    rms = torch.sqrt((h * h).mean(-1, keepdim=True) + 1e-6)
    return ((h / rms) * i["weight"].float()).to(i["x"].dtype)


def _scan_inputs(s, dt, dev, seed):
    g = _gen(seed, dev)
    b, d, n, l = s["batch"], s["dim"], s["dstate"], s["seqlen"]
    return {"u": torch.randn(b, d, l, device=dev, generator=g).to(dt),
            "delta": (0.5 * torch.rand(b, d, l, device=dev, generator=g)).to(dt),
            "A": -0.5 * torch.rand(d, n, device=dev, generator=g),
            "B": torch.randn(b, n, l, device=dev, generator=g).to(dt),
            "C": torch.randn(b, n, l, device=dev, generator=g).to(dt),
            "D": torch.randn(d, device=dev, generator=g),
            "z": torch.randn(b, d, l, device=dev, generator=g).to(dt)}


def _scan_ref(i):
    """selective_scan_ref (selective_scan_interface.py:115-181) step by step in
    fp32, delta' = softplus(delta), gate silu(z) in fp32."""
    u, A, D = i["u"].float(), i["A"], i["D"]
    dl = F.softplus(i["delta"].float())
    Bm, Cm = i["B"].float(), i["C"].float()
    h = torch.zeros(u.shape[0], u.shape[1], A.shape[1], device=u.device)
    ys = []
    for t in range(u.shape[2]):
        h = torch.exp(dl[:, :, t, None] * A) * h + (dl[:, :, t] * u[:, :, t])[..., None] * Bm[:, None, :, t]
        ys.append((h * Cm[:, None, :, t]).sum(-1))
    y = torch.stack(ys, dim=2) + u * D[:, None]
    return (y * F.silu(i["z"].float())).to(i["u"].dtype)


def _scan_kernel(u, delta, A, B, C, D, z):
    from kernels.hip.selective_scan import selective_scan_fn
    return selective_scan_fn(u, delta, A, B, C, D, z, None, True)


def _kernels():
    from kernels import ce_fused
    from kernels.hip import fused_residual_add_rmsnorm, rmsnorm, softmax
    return {"softmax": softmax.kernel_fn, "cross_entropy": ce_fused.kernel_fn,
            "rmsnorm": rmsnorm.kernel_fn, "fused_residual_add_rmsnorm": fused_residual_add_rmsnorm.kernel_fn,
            "selective_scan": _scan_kernel}


def _specs() -> Dict[str, KernelSpec]:
    k = _kernels()
    half = {torch.float16: {"atol": 1e-2, "rtol": 1e-2}, torch.bfloat16: {"atol": 2e-2, "rtol": 2e-2},
            torch.float32: {"atol": 1e-5, "rtol": 1e-5}}
    return {
        "softmax": KernelSpec(
            "softmax",
            [("tiny", {"rows": 32, "cols": 128}), ("small", {"rows": 256, "cols": 512}),
             ("medium", {"rows": 1024, "cols": 1024}), ("large", {"rows": 4096, "cols": 4096}),
             ("xlarge", {"rows": 8192, "cols": 8192}), ("wide", {"rows": 1024, "cols": 32768}),
             ("narrow", {"rows": 32768, "cols": 128}), ("vocab", {"rows": 4096, "cols": 50257}),
             ("c2", {"rows": 98304, "cols": 1024})],
            [torch.float16, torch.bfloat16, torch.float32],
            {torch.float16: {"atol": 1e-3, "rtol": 1e-3}, torch.bfloat16: {"atol": 2e-3, "rtol": 2e-3},
             torch.float32: {"atol": 1e-5, "rtol": 1e-5}},
            _softmax_inputs, _softmax_ref, k["softmax"],
            lambda s: 5 * s["rows"] * s["cols"],
            lambda s, dt: 2 * s["rows"] * s["cols"] * _esize(dt),
            [("edge_1023", {"rows": 1023, "cols": 1023}), ("edge_4097", {"rows": 4097, "cols": 4097}),
             ("edge_50257", {"rows": 1024, "cols": 50257})]),
        "cross_entropy": KernelSpec(
            "cross_entropy",
            [("tiny", {"batch": 32, "vocab": 256}), ("small", {"batch": 256, "vocab": 1024}),
             ("medium", {"batch": 1024, "vocab": 4096}), ("large", {"batch": 4096, "vocab": 32000}),
             ("xlarge", {"batch": 8192, "vocab": 50257}), ("gpt2", {"batch": 4096, "vocab": 50257})],
            [torch.float16, torch.bfloat16, torch.float32], dict(half),
            _ce_inputs, _ce_ref, k["cross_entropy"],
            lambda s: 4 * s["batch"] * s["vocab"],
            lambda s, dt: (s["batch"] * s["vocab"] + s["batch"]) * _esize(dt),
            [("edge_1023", {"batch": 1023, "vocab": 32000}), ("edge_50257", {"batch": 4096, "vocab": 50257})]),
        "rmsnorm": KernelSpec(
            "rmsnorm",
            [("small", {"M": 1024, "N": 768}), ("medium", {"M": 4096, "N": 1024}),
             ("large", {"M": 4096, "N": 4096}), ("llama", {"M": 2048, "N": 4096}),
             ("c1", {"M": 2048, "N": 768})],
            [torch.float16, torch.bfloat16, torch.float32],
            {torch.float16: {"atol": 1e-2, "rtol": 1e-2}, torch.bfloat16: {"atol": 1e-1, "rtol": 5e-2},
             torch.float32: {"atol": 1e-5, "rtol": 1e-5}},
            _rms_inputs, _rms_ref, k["rmsnorm"],
            lambda s: 6 * s["M"] * s["N"],
            lambda s, dt: (2 * s["M"] * s["N"] + s["N"]) * _esize(dt),
            [("edge_1023", {"M": 1023, "N": 768}), ("edge_4097", {"M": 4097, "N": 1024})]),
        "fused_residual_add_rmsnorm": KernelSpec(
            "fused_residual_add_rmsnorm",
            [("small", {"M": 1024, "N": 768}), ("medium", {"M": 4096, "N": 1024}),
             ("large", {"M": 4096, "N": 4096}), ("llama", {"M": 2048, "N": 4096}),
             ("c3", {"M": 16384, "N": 4096})],
            [torch.float16, torch.bfloat16, torch.float32],
            {torch.float16: {"atol": 1e-2, "rtol": 1e-2}, torch.bfloat16: {"atol": 1e-1, "rtol": 5e-2},
             torch.float32: {"atol": 1e-5, "rtol": 1e-5}},
            _fused_inputs, _fused_ref, k["fused_residual_add_rmsnorm"],
            lambda s: 7 * s["M"] * s["N"],
            lambda s, dt: (3 * s["M"] * s["N"] + s["N"]) * _esize(dt),
            [("edge_1023", {"M": 1023, "N": 768}), ("edge_4097", {"M": 4097, "N": 1024})]),
        "selective_scan": KernelSpec(
            "selective_scan",
            [("tiny", {"batch": 1, "dim": 16, "dstate": 16, "seqlen": 64}),
             ("small", {"batch": 2, "dim": 64, "dstate": 16, "seqlen": 256}),
             ("large", {"batch": 4, "dim": 512, "dstate": 16, "seqlen": 1024}),
             ("n64", {"batch": 8, "dim": 384, "dstate": 64, "seqlen": 512})],
            [torch.bfloat16, torch.float16, torch.float32],
            {torch.bfloat16: {"atol": 5e-2, "rtol": 3e-2}, torch.float16: {"atol": 5e-3, "rtol": 3e-3},
             torch.float32: {"atol": 2e-3, "rtol": 6e-4}},
            _scan_inputs, _scan_ref, k["selective_scan"],
            lambda s: 7 * s["batch"] * s["dim"] * s["dstate"] * s["seqlen"],
            lambda s, dt: (4 * s["batch"] * s["dim"] * s["seqlen"] + 2 * s["batch"] * s["dstate"] * s["seqlen"])
            * _esize(dt),
            [("edge_127", {"batch": 1, "dim": 33, "dstate": 7, "seqlen": 127}),
             ("edge_wide", {"batch": 1, "dim": 20, "dstate": 48, "seqlen": 100})],
            primary="large", adversarial=False),
    }


class _Configs(dict):
    """KERNEL_CONFIGS, built on first use (kernel modules load the library)."""

    def _fill(self):
        if not dict.__len__(self):
            self.update(_specs())

    def __getitem__(self, key):
        self._fill()
        return dict.__getitem__(self, key)

    def __contains__(self, key):
        self._fill()
        return dict.__contains__(self, key)

    def __iter__(self):
        self._fill()
        return dict.__iter__(self)

    def keys(self):
        self._fill()
        return dict.keys(self)


KERNEL_CONFIGS: Dict[str, KernelSpec] = _Configs()


# ---------------------------------------------------------------------------
# Comparison
# ---------------------------------------------------------------------------

def _nonfinite(t: torch.Tensor) -> bool:
    return not bool(torch.isfinite(t.float()).all())


def compare(out: torch.Tensor, ref: torch.Tensor, atol: float, rtol: float) -> dict:
    """Shape, elementwise |out - ref| <= atol + rtol |ref| (NaN where both are
    NaN counts as a match), max / mean absolute error, % within tolerance."""
    if out.shape != ref.shape:
        return {"match": False, "reason": f"shape {tuple(out.shape)} != {tuple(ref.shape)}",
                "max_abs_error": math.inf, "pct_within_tol": 0.0}
    o, r = out.detach().float(), ref.detach().float()
    both_nan = torch.isnan(o) & torch.isnan(r)
    diff = torch.where(both_nan, torch.zeros_like(o), (o - r).abs())
    same_inf = torch.isinf(o) & (o == r)
    ok = (diff <= atol + rtol * r.abs()) | both_nan | same_inf
    diff = torch.where(same_inf, torch.zeros_like(diff), diff)
    max_err = float(torch.nan_to_num(diff, nan=math.inf).max()) if diff.numel() else 0.0
    match = bool(ok.all())
    return {"match": match, "max_abs_error": max_err,
            "pct_within_tol": float(ok.float().mean() * 100) if ok.numel() else 100.0,
            "reason": "" if match else f"max_abs_error={max_err:.3e} exceeds atol={atol}, rtol={rtol}"}


# ---------------------------------------------------------------------------
# Correctness: five stages
# ---------------------------------------------------------------------------

ADVERSARIAL = (
    ("near_max", lambda t: t * (60000.0 if t.dtype == torch.float16 else 1e30)),
    ("near_zero", lambda t: t * 1e-6),
    ("mixed_scale", lambda t: t * torch.where(torch.rand(t.shape, device=t.device,
                                                         generator=_gen(7, str(t.device))) > 0.5,
                                              1e3, 1e-3).to(t.dtype)),
    ("all_zeros", lambda t: torch.zeros_like(t)),
    ("all_same", lambda t: torch.full_like(t, 0.5)),
)


def _run(spec: KernelSpec, inputs: dict) -> torch.Tensor:
    out = spec.kernel_fn(**inputs)
    torch.cuda.synchronize()
    return out


def run_correctness(spec: KernelSpec, quick: bool = False, device: str = "cuda",
                    log=print) -> dict:
    """The reference's five correctness stages for one kernel type. Returns
    ``{stage: "PASS ..." | "FAIL ..." | "SKIP ...", "correctness": PASS|FAIL,
    "details": [...]}``."""
    res = {"smoke_test": "SKIP", "shape_sweep": "SKIP", "numerical_stability": "SKIP",
           "determinism": "SKIP", "edge_cases": "SKIP", "correctness": "FAIL", "details": []}
    ok_all = True
    tol = lambda dt: spec.tolerances.get(dt, {"atol": 1e-2, "rtol": 1e-2})

    def check(label, size, dt, relax=1.0):
        inputs = spec.input_generator(size, dt, device, 42)
        expected = spec.reference_fn(inputs)
        out = _run(spec, inputs)
        if _nonfinite(out) and not _nonfinite(expected):
            return False, f"{label}: NaN/Inf where the reference is finite", 0.0
        t = tol(dt)
        c = compare(out, expected, t["atol"] * relax, t["rtol"] * relax)
        return c["match"], (f"{label}: " + c["reason"]) if not c["match"] else "", c["max_abs_error"]

    # Stage 1: smoke test
    log("\n--- Stage 1: Smoke Test ---")
    label, size = spec.test_sizes[0]
    try:
        ok, why, err = check(label, size, spec.test_dtypes[0])
        res["smoke_test"] = "PASS" if ok else "FAIL"
        log(f"  {'PASS' if ok else 'FAIL'} (max_abs_error={err:.6e}) {why}")
        if not ok:
            res["details"].append(why)
    except Exception as e:  # a crash fails the stage, as in the reference harness
        res["smoke_test"] = "FAIL"
        res["details"].append(f"smoke: CRASH ({type(e).__name__}: {e})")
        log(f"  FAIL: CRASH ({type(e).__name__}: {e})")
    if res["smoke_test"] != "PASS":
        log("\ncorrectness: FAIL (smoke test failed, remaining stages skipped)")
        return res

    # Stage 2: every size x dtype
    log("\n--- Stage 2: Shape Sweep ---")
    n, bad, worst, worst_at = 0, 0, 0.0, ""
    for label, size in spec.test_sizes:
        for dt in spec.test_dtypes:
            n += 1
            try:
                ok, why, err = check(label, size, dt)
            except torch.cuda.OutOfMemoryError:
                log(f"  SKIP: {label} {dt} (out of memory)")
                torch.cuda.empty_cache()
                continue
            except Exception as e:
                ok, why, err = False, f"{label}/{dt}: {type(e).__name__}: {e}", 0.0
            if err > worst:
                worst, worst_at = err, f"{label}/{dt}"
            log(f"  {'PASS' if ok else 'FAIL'}: {label} {dt} (max_err={err:.2e}) {why}")
            if not ok:
                bad += 1
                res["details"].append(why)
    if bad:
        res["shape_sweep"] = f"FAIL ({bad}/{n} failed)"
        ok_all = False
    else:
        res["shape_sweep"] = f"PASS ({n} configs, worst_err={worst:.2e} at {worst_at})"
    log(f"  shape_sweep: {res['shape_sweep']}")

    if quick:
        for k in ("numerical_stability", "determinism", "edge_cases"):
            res[k] = "SKIP (quick mode)"
        res["correctness"] = "PASS" if ok_all else "FAIL"
        log(f"\ncorrectness: {res['correctness']} (quick mode: stages 3-5 skipped)")
        return res

    # Stage 3: adversarial inputs on the "small" size (tolerances x 10)
    log("\n--- Stage 3: Numerical Stability ---")
    small = dict(spec.test_sizes).get("small", spec.test_sizes[min(1, len(spec.test_sizes) - 1)][1])
    stab_ok = True
    for name, fn in (ADVERSARIAL if spec.adversarial else ()):
        try:
            inputs = spec.input_generator(small, spec.test_dtypes[0], device, 42)
            inputs = {k: fn(v) if isinstance(v, torch.Tensor) and v.is_floating_point() else v
                      for k, v in inputs.items()}
            expected = spec.reference_fn(inputs)
            out = _run(spec, inputs)
            if _nonfinite(out) and _nonfinite(expected):
                # both overflow: the non-finite pattern must agree
                same = bool(((torch.isnan(out.float()) == torch.isnan(expected.float()))
                             & (torch.isinf(out.float()) == torch.isinf(expected.float()))).all())
                log(f"  {'PASS' if same else 'FAIL'}: {name} (both non-finite)")
                if not same:
                    stab_ok = False
                    res["details"].append(f"stability {name}: different NaN/Inf pattern")
                continue
            if _nonfinite(out):
                stab_ok = False
                res["details"].append(f"stability {name}: NaN/Inf where the reference is finite")
                log(f"  FAIL: {name} (NaN/Inf, reference finite)")
                continue
            t = tol(spec.test_dtypes[0])
            c = compare(out, expected, 10 * t["atol"], 10 * t["rtol"])
            log(f"  {'PASS' if c['match'] else 'FAIL'}: {name} (max_err={c['max_abs_error']:.2e})")
            if not c["match"]:
                stab_ok = False
                res["details"].append(f"stability {name}: {c['reason']}")
        except Exception as e:
            stab_ok = False
            res["details"].append(f"stability {name}: {type(e).__name__}: {e}")
            log(f"  FAIL: {name} ({type(e).__name__}: {e})")
    res["numerical_stability"] = ("PASS" if stab_ok else "FAIL") if spec.adversarial else \
        "SKIP (no adversarial transforms defined for this kernel)"
    ok_all &= stab_ok
    log(f"  numerical_stability: {res['numerical_stability']}")

    # Stage 4: three runs, bitwise identical
    log("\n--- Stage 4: Determinism ---")
    try:
        outs = [_run(spec, spec.input_generator(small, spec.test_dtypes[0], device, 42)) for _ in range(3)]
        det = all(torch.equal(outs[0], o) for o in outs[1:])
    except Exception as e:
        det = False
        res["details"].append(f"determinism: {type(e).__name__}: {e}")
    res["determinism"] = "PASS" if det else "FAIL"
    ok_all &= det
    log(f"  {'PASS: 3 runs are bitwise identical' if det else 'FAIL'}")

    # Stage 5: sizes off the power-of-two grid
    log("\n--- Stage 5: Edge Cases ---")
    if not spec.edge_sizes:
        res["edge_cases"] = "SKIP (no edge sizes defined)"
    else:
        edge_ok = True
        for label, size in spec.edge_sizes:
            try:
                ok, why, err = check(label, size, spec.test_dtypes[0])
            except Exception as e:
                ok, why, err = False, f"{label}: {type(e).__name__}: {e}", 0.0
            log(f"  {'PASS' if ok else 'FAIL'}: {label} (max_err={err:.2e}) {why}")
            if not ok:
                edge_ok = False
                res["details"].append(why)
        res["edge_cases"] = "PASS" if edge_ok else "FAIL"
        ok_all &= edge_ok
    log(f"  edge_cases: {res['edge_cases']}")

    res["correctness"] = "PASS" if ok_all else "FAIL"
    log(f"\ncorrectness: {res['correctness']}")
    return res


# ---------------------------------------------------------------------------
# Performance
# ---------------------------------------------------------------------------

def median_launch_ms(fn: Callable[[], object], reps: int = 100, warmup: int = 10) -> float:
    """Median over ``reps`` launches of the time between an event pair recorded
    on the current stream around each launch.

    The pairs are issued while a spin kernel holds the stream (about 1 ms,
    doubled while the GPU still drains the queue before the host is done), so
    that launches shorter than their host issue time are timed on the GPU."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    hold = 2_000_000
    while True:
        pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                 for _ in range(reps)]
        torch.cuda._sleep(hold)
        for a, b in pairs:
            a.record()
            fn()
            b.record()
        drained = pairs[-1][1].query()
        torch.cuda.synchronize()
        if not drained or hold >= 16_000_000:
            break
        hold *= 2
    ts = sorted(a.elapsed_time(b) for a, b in pairs)
    return ts[len(ts) // 2]


def run_performance(spec: KernelSpec, sizes: str = "all", device: str = "cuda",
                    reps: int = 100, log=print) -> dict:
    """Median kernel and eager-PyTorch times per size (first dtype), with
    throughput, bandwidth and fractions of the MI355X peaks. The primary size
    is ``spec.primary`` (or the last one)."""
    chosen = spec.test_sizes if sizes == "all" else [s for s in spec.test_sizes if s[0] == sizes]
    if not chosen:
        chosen = [s for s in spec.test_sizes if s[0] == spec.primary] or [spec.test_sizes[-1]]
    dt = spec.test_dtypes[0]
    rows, primary = [], None
    ridge = PEAK_TFLOPS_16 * 1e12 / (PEAK_HBM_GBS * 1e9)
    for label, size in chosen:
        log(f"\n  Benchmarking: {label} ...")
        inputs = spec.input_generator(size, dt, device, 42)
        k_ms = median_launch_ms(lambda: spec.kernel_fn(**inputs), reps)
        r_ms = median_launch_ms(lambda: spec.reference_fn(inputs), min(reps, 20) if label == "large"
                                and spec.kernel_type == "selective_scan" else reps)
        flops, nbytes = spec.flops_fn(size), spec.bytes_fn(size, dt)
        tf = flops / (k_ms * 1e-3) / 1e12
        gbs = nbytes / (k_ms * 1e-3) / 1e9
        ai = flops / nbytes if nbytes else 0.0
        e = {"label": label, "size": size, "dtype": str(dt), "flops": flops, "bytes": nbytes,
             "kernel_latency_us": k_ms * 1e3, "pytorch_latency_us": r_ms * 1e3,
             "throughput_tflops": tf, "bandwidth_gb_s": gbs,
             "ref_throughput_tflops": flops / (r_ms * 1e-3) / 1e12,
             "pct_peak_compute": 100 * tf / PEAK_TFLOPS_16, "pct_peak_bandwidth": 100 * gbs / PEAK_HBM_GBS,
             "arithmetic_intensity": ai, "ridge_point": ridge,
             "bottleneck": "memory_bound" if ai < ridge else "compute_bound",
             "speedup_vs_pytorch": r_ms / k_ms}
        rows.append(e)
        log(f"    kernel {e['kernel_latency_us']:.2f} us, pytorch {e['pytorch_latency_us']:.2f} us, "
            f"{gbs:.1f} GB/s ({e['pct_peak_bandwidth']:.1f}% of HBM peak), speedup {e['speedup_vs_pytorch']:.3f}x")
        if label == spec.primary:
            primary = e
    return {"primary": primary or rows[-1], "all": rows}


# ---------------------------------------------------------------------------
# Report
# ---------------------------------------------------------------------------

def main(argv: Optional[List[str]] = None, log=print) -> dict:
    """The reference harness's run and report for one kernel type; returns the
    correctness and performance results."""
    t0 = time.time()
    ap = argparse.ArgumentParser(description="gfx950 kernel harness")
    ap.add_argument("--kernel", default=None, help="kernel type (default: kernel.py's KERNEL_TYPE)")
    ap.add_argument("--sizes", default="all", help="size label to time, or all")
    ap.add_argument("--quick", action="store_true", help="skip correctness stages 3-5, time 'large' only")
    ap.add_argument("--reps", type=int, default=100)
    a = ap.parse_args(argv)
    kernel_type = a.kernel
    if kernel_type is None:
        import kernel
        kernel_type = kernel.KERNEL_TYPE
    log("=" * 60)
    log("AutoKernel gfx950 harness")
    log("=" * 60)
    log(f"kernel_type: {kernel_type}")
    if kernel_type not in KERNEL_CONFIGS:
        log(f"ERROR: unknown kernel type {kernel_type!r}; available: {', '.join(KERNEL_CONFIGS.keys())}")
        log("\ncorrectness: FAIL")
        log("throughput_tflops: 0.000")
        return {"correctness": {"correctness": "FAIL"}, "performance": None}
    spec = KERNEL_CONFIGS[kernel_type]

    p = torch.cuda.get_device_properties(0)
    log("\n=== GPU INFO ===")
    log(f"gpu_name: {p.name}")
    log(f"gpu_arch: {getattr(p, 'gcnArchName', 'unknown')}")
    log(f"gpu_cu_count: {p.multi_processor_count}")
    log(f"gpu_memory_gb: {p.total_memory / 2**30:.1f}")
    log(f"gpu_peak_tflops_bf16: {PEAK_TFLOPS_16}")
    log(f"gpu_peak_bandwidth_gb_s: {PEAK_HBM_GBS}")

    log("\n=== CORRECTNESS ===")
    corr = run_correctness(spec, quick=a.quick, log=log)
    log("\n--- Correctness Summary ---")
    for k in ("smoke_test", "shape_sweep", "numerical_stability", "determinism", "edge_cases",
              "correctness"):
        log(f"{k}: {corr[k]}")

    perf = None
    try:
        perf = run_performance(spec, "large" if a.quick and a.sizes == "all" else a.sizes,
                               reps=a.reps, log=log)
    except Exception as e:  # timing failures are reported, not raised
        log(f"\nperformance failed: {type(e).__name__}: {e}")
    prim = perf["primary"] if perf else None
    if prim:
        log(f"\n=== PERFORMANCE ({prim['label']}: "
            f"{', '.join(f'{k}={v}' for k, v in prim['size'].items())}, dtype={prim['dtype']}) ===")
        for k in ("kernel_latency_us", "throughput_tflops", "bandwidth_gb_s", "pct_peak_compute",
                  "pct_peak_bandwidth", "arithmetic_intensity", "bottleneck"):
            v = prim[k]
            log(f"{k}: {v:.3f}" if isinstance(v, float) else f"{k}: {v}")
        log("\n=== COMPARISON VS PYTORCH ===")
        log(f"pytorch_latency_us: {prim['pytorch_latency_us']:.2f}")
        log(f"kernel_latency_us: {prim['kernel_latency_us']:.2f}")
        log(f"speedup_vs_pytorch: {prim['speedup_vs_pytorch']:.3f}x")
    if perf and len(perf["all"]) > 1:
        log("\n=== SIZE SWEEP ===")
        log(f"{'size':<12} {'kernel_us':>12} {'pytorch_us':>12} {'speedup':>10} {'GB/s':>10} {'%hbm':>8}")
        for e in perf["all"]:
            log(f"{e['label']:<12} {e['kernel_latency_us']:>12.2f} {e['pytorch_latency_us']:>12.2f} "
                f"{e['speedup_vs_pytorch']:>9.3f}x {e['bandwidth_gb_s']:>10.1f} {e['pct_peak_bandwidth']:>7.1f}%")

    log("\n=== FINAL ===")
    log(f"kernel_type: {kernel_type}")
    log(f"correctness: {corr['correctness']}")
    log(f"throughput_tflops: {prim['throughput_tflops'] if prim else 0.0:.3f}")
    log(f"speedup_vs_pytorch: {prim['speedup_vs_pytorch'] if prim else 0.0:.3f}x")
    log(f"pct_peak_compute: {prim['pct_peak_compute'] if prim else 0.0:.1f}%")
    log(f"pct_peak_bandwidth: {prim['pct_peak_bandwidth'] if prim else 0.0:.1f}%")
    log(f"bench_time_seconds: {time.time() - t0:.1f}")
    return {"correctness": corr, "performance": perf}


if __name__ == "__main__":
    out = main(sys.argv[1:])
    sys.exit(0 if out["correctness"]["correctness"] == "PASS" else 1)
