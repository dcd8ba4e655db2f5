"""Model-level verification with the gfx950 kernels swapped in.

The counterpart of the reference's ``verify.py`` model check
(``OptimizedModelContext`` :809-900, ``compare_outputs`` :1152-1230): a
context manager replaces a model's RMSNorm modules and pre-norm blocks with
modules that call the gfx950 kernels, the model runs once without and once
with them, and the outputs are compared at dtype tolerances. Leaving the
context restores every original module object.

Kernel types with a replacement here: ``rmsnorm`` (RMSNorm-like modules:
the reference's class names, or a module with ``weight`` and ``eps`` and no
``bias`` whose class name ends in ``norm``, :939-968) and
``fused_residual_add_rmsnorm`` (pre-norm blocks with attention,
attention_norm, feed_forward and ffn_norm, or the other attribute families
of ``autokernel._patterns``, :1033-1050). The reference's other types
(matmul, layernorm, silu_gate_mul, rotary_embedding, fused_qkv) are outside
this kernel set and are skipped with a note, as the reference does for types
it has no strategy for.
"""

from __future__ import annotations

import importlib
import time
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Optional

import torch
import torch.nn as nn

DEFAULT_TOLERANCES = {
    torch.float32: {"atol": 1e-4, "rtol": 1e-4},
    torch.float16: {"atol": 1e-2, "rtol": 1e-2},
    torch.bfloat16: {"atol": 2e-2, "rtol": 2e-2},
}

# kernel type -> the module whose entry point the replacement calls
KERNEL_MODULES = {
    "rmsnorm": "kernels.hip.rmsnorm",
    "fused_residual_add_rmsnorm": "kernels.hip.fused_residual_add_rmsnorm",
}

_RMSNORM_NAMES = {"RMSNorm", "LlamaRMSNorm", "T5LayerNorm", "GemmaRMSNorm"}


@dataclass
class KernelReplacement:
    """One kernel to swap in: its type, the profiling rank and speedup it was
    chosen with, and where its entry point lives (a module path such as
    ``kernels.hip.rmsnorm``; empty for the built-in kernel of the type)."""
    kernel_type: str
    rank: int = 0
    speedup: float = 1.0
    optimized_path: str = ""
    module_fn: Optional[Callable] = None


def load_kernel_module(path: str) -> Any:
    """Import a kernel module by dotted path."""
    return importlib.import_module(path)


def _is_rmsnorm(module: nn.Module) -> bool:
    name = type(module).__name__
    if name in _RMSNORM_NAMES or isinstance(module, getattr(nn, "RMSNorm", ())):
        return True
    return (hasattr(module, "weight") and hasattr(module, "eps") and not hasattr(module, "bias")
            and name.lower().endswith("norm") and not isinstance(module, nn.LayerNorm))


class OptimizedModelContext:
    """``with OptimizedModelContext(model, replacements) as m: m(x)`` runs the
    model with the gfx950 kernels in place of its RMSNorm modules and / or
    pre-norm blocks; the originals are restored on exit. ``applied`` lists what
    was replaced."""

    def __init__(self, model: nn.Module, replacements: List[KernelReplacement],
                 fused_qkv: bool = False,
                 all_replacements: Optional[List[KernelReplacement]] = None):
        self.model = model
        self.replacements = replacements
        self.fused_qkv = fused_qkv
        self._all_replacements = all_replacements or replacements
        # (parent module, attribute, original module), in replacement order
        self._undo: List[tuple] = []
        self.applied: List[str] = []
        self.notes: List[str] = []

    # -- entry points ------------------------------------------------------
    def _entry(self, repl: KernelReplacement) -> Optional[Callable]:
        path = repl.optimized_path or KERNEL_MODULES.get(repl.kernel_type, "")
        if not path:
            return None
        mod = load_kernel_module(path)
        want = "kernel_fn_dual" if repl.kernel_type == "fused_residual_add_rmsnorm" else "kernel_fn"
        return getattr(mod, want, None)

    def __enter__(self) -> nn.Module:
        if self.fused_qkv:
            self.notes.append("fused_qkv: outside this kernel set, not applied")
        for repl in sorted(self.replacements, key=lambda r: r.rank):
            if repl.kernel_type not in KERNEL_MODULES:
                self.notes.append(f"{repl.kernel_type}: no replacement strategy in this kernel set, skipped")
                continue
            fn = self._entry(repl)
            if fn is None:
                self.notes.append(f"{repl.kernel_type}: {repl.optimized_path} has no entry point, skipped")
                continue
            repl.module_fn = fn
            n = (self._swap_blocks(fn) if repl.kernel_type == "fused_residual_add_rmsnorm"
                 else self._swap_norms(fn))
            if n:
                self.applied.append(f"{repl.kernel_type} (rank {repl.rank}): {n} modules, "
                                    f"{repl.speedup:.1f}x")
        return self.model

    def __exit__(self, *exc) -> None:
        # undo in reverse order: a norm swapped inside an original block is
        # restored after that block is back in place
        while self._undo:
            parent, attr, original = self._undo.pop()
            setattr(parent, attr, original)

    # -- swapping ----------------------------------------------------------
    def _replace(self, name: str, original: nn.Module, new: nn.Module) -> None:
        if name == "":
            raise ValueError("the model itself cannot be replaced")
        parent = self.model
        *path, leaf = name.split(".")
        for p in path:
            parent = getattr(parent, p)
        self._undo.append((parent, leaf, original))
        setattr(parent, leaf, new)

    def _swap_norms(self, fn: Callable) -> int:
        from autokernel._patterns import _RMSNormReplacement
        count = 0
        for name, module in list(self.model.named_modules()):
            if name and _is_rmsnorm(module) and not isinstance(module, _RMSNormReplacement):
                self._replace(name, module, _RMSNormReplacement(module, fn))
                count += 1
        return count

    def _swap_blocks(self, fn_dual: Callable) -> int:
        from autokernel._patterns import _FusedResidualRMSNormBlockReplacement, _find_block_attrs
        count = 0
        for name, module in list(self.model.named_modules()):
            attrs = _find_block_attrs(module) if name else None
            if attrs is not None:
                self._replace(name, module, _FusedResidualRMSNormBlockReplacement(module, fn_dual, *attrs))
                count += 1
        return count


def compare_outputs(ref_output: torch.Tensor, opt_output: torch.Tensor, dtype: torch.dtype,
                    custom_atol: Optional[float] = None, custom_rtol: Optional[float] = None) -> Dict[str, Any]:
    """Shape, NaN / Inf and tolerance comparison of two model outputs
    (``correctness``: PASS / FAIL, with ``reason`` on failure)."""
    r: Dict[str, Any] = {"shapes_match": ref_output.shape == opt_output.shape,
                         "ref_shape": list(ref_output.shape), "opt_shape": list(opt_output.shape)}
    if not r["shapes_match"]:
        r.update(correctness="FAIL", reason=f"shape mismatch: ref={r['ref_shape']}, opt={r['opt_shape']}")
        return r
    a, b = ref_output.detach().float(), opt_output.detach().float()
    for tag, t in (("ref", a), ("opt", b)):
        r[f"{tag}_has_nan"] = bool(torch.isnan(t).any())
        r[f"{tag}_has_inf"] = bool(torch.isinf(t).any())
    if r["opt_has_nan"] and not r["ref_has_nan"]:
        r.update(correctness="FAIL", reason="optimized output has NaN where the reference has none")
        return r
    if r["opt_has_inf"] and not r["ref_has_inf"]:
        r.update(correctness="FAIL", reason="optimized output has Inf where the reference has none")
        return r
    keep = ~(torch.isnan(a) & torch.isnan(b))
    diff = (a - b).abs()[keep]
    r["max_abs_error"] = float(diff.max()) if diff.numel() else 0.0
    r["mean_abs_error"] = float(diff.mean()) if diff.numel() else 0.0
    tol = DEFAULT_TOLERANCES.get(dtype, {"atol": 1e-4, "rtol": 1e-4})
    atol = tol["atol"] if custom_atol is None else custom_atol
    rtol = tol["rtol"] if custom_rtol is None else custom_rtol
    ok = bool(torch.allclose(a[keep], b[keep], atol=atol, rtol=rtol)) if diff.numel() else True
    r.update(correctness="PASS" if ok else "FAIL", atol=atol, rtol=rtol)
    if not ok:
        r["reason"] = (f"values exceed tolerance (atol={atol}, rtol={rtol}): "
                       f"max_abs_error={r['max_abs_error']:.6e}, mean_abs_error={r['mean_abs_error']:.6e}")
    return r


@dataclass
class VerificationResult:
    """Outcome of :func:`verify_model`."""
    input_shape: str = ""
    dtype_str: str = ""
    ref_latency_ms: float = 0.0
    opt_latency_ms: float = 0.0
    kernels_replaced: List[str] = field(default_factory=list)
    notes: List[str] = field(default_factory=list)
    comparison: Dict[str, Any] = field(default_factory=dict)

    @property
    def correctness(self) -> str:
        return self.comparison.get("correctness", "FAIL")

    @property
    def speedup(self) -> float:
        return self.ref_latency_ms / self.opt_latency_ms if self.opt_latency_ms else 0.0


def _timed(model: nn.Module, args: tuple, reps: int) -> tuple:
    with torch.no_grad():
        out = model(*args)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            model(*args)
        torch.cuda.synchronize()
    return out, (time.perf_counter() - t0) * 1e3 / max(reps, 1)


def verify_model(model: nn.Module, example_args: tuple, replacements: List[KernelReplacement],
                 dtype: Optional[torch.dtype] = None, reps: int = 5,
                 atol: Optional[float] = None, rtol: Optional[float] = None) -> VerificationResult:
    """Runs ``model(*example_args)`` as is and inside :class:`OptimizedModelContext`
    and compares the outputs (the first tensor of a tuple output)."""
    dtype = dtype or next(model.parameters()).dtype
    first = lambda o: o[0] if isinstance(o, (tuple, list)) else o
    ref, ref_ms = _timed(model, example_args, reps)
    ctx = OptimizedModelContext(model, replacements)
    with ctx as m:
        opt, opt_ms = _timed(m, example_args, reps)
        applied, notes = list(ctx.applied), list(ctx.notes)
    res = VerificationResult(
        input_shape=str([list(a.shape) for a in example_args if isinstance(a, torch.Tensor)]),
        dtype_str=str(dtype), ref_latency_ms=ref_ms, opt_latency_ms=opt_ms,
        kernels_replaced=applied, notes=notes,
        comparison=compare_outputs(first(ref), first(opt), dtype, atol, rtol))
    return res
