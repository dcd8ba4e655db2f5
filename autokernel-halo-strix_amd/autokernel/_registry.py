"""Pattern matching and module replacement for ``autokernel.optimize``.

Behaviour of the reference ``autokernel/_registry.py:64-178``: optionally cast
the model (complex buffers preserved), move it to the GPU, apply patterns in
descending priority over ``named_modules()`` (a module replaced by a
higher-priority pattern is not matched again), keep the originals so
``restore`` can undo the swap, and record counts for ``report``.
``compile=True`` wraps the result in ``torch.compile`` (the custom ops have
fake implementations, so they trace as opaque nodes).
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional, Set

import torch
import torch.nn as nn

from autokernel._patterns import ALL_PATTERNS, Pattern

_STATE_ATTR = "_autokernel_state"


def _replace_module(model: nn.Module, name: str, new_module: nn.Module) -> None:
    parent = model
    parts = name.split(".")
    for p in parts[:-1]:
        parent = getattr(parent, p)
    setattr(parent, parts[-1], new_module)


def _complex_buffers(model: nn.Module) -> Dict[str, torch.Tensor]:
    return {n: b.clone() for n, b in model.named_buffers() if b.is_complex()}


def _put_back_buffers(model: nn.Module, saved: Dict[str, torch.Tensor]) -> None:
    device = next(model.parameters()).device
    for name, buf in saved.items():
        parent = model
        parts = name.split(".")
        for p in parts[:-1]:
            parent = getattr(parent, p)
        parent.register_buffer(parts[-1], buf.to(device), persistent=False)


def _select_patterns(include: Optional[List[str]], exclude: Optional[List[str]]) -> List[Pattern]:
    patterns = list(ALL_PATTERNS)
    if include is not None:
        keep = set(include)
        patterns = [p for p in patterns if p.name in keep]
    if exclude is not None:
        drop = set(exclude)
        patterns = [p for p in patterns if p.name not in drop]
    return patterns


def optimize(model: nn.Module, dtype: torch.dtype = torch.float16, compile: bool = False,
             compile_mode: str = "default", include: Optional[List[str]] = None,
             exclude: Optional[List[str]] = None, training: bool = False) -> nn.Module:
    """Apply every matching pattern to ``model`` in place and return it.

    ``training=True`` leaves parameter dtypes alone (AMP casts at run time)
    and keeps the model in train mode.
    """
    if not training:
        saved = _complex_buffers(model)
        model = model.to(dtype=dtype)
        if saved:
            _put_back_buffers(model, saved)
    params = list(model.parameters())
    if torch.cuda.is_available() and params and not params[0].is_cuda:
        model = model.cuda()
    if not training:
        model.eval()

    patterns = sorted(_select_patterns(include, exclude), key=lambda p: -p.priority)
    originals: Dict[str, nn.Module] = {}
    applied: Dict[str, int] = {}
    replaced: Set[str] = set()
    for pattern in patterns:
        count = 0
        for name, module in list(model.named_modules()):
            if name in replaced or not name:
                continue
            if pattern.matches(name, module, model):
                try:
                    replacement = pattern.apply(name, module, model)
                except Exception as e:  # a failed swap leaves the module untouched
                    print(f"  autokernel: {pattern.name} failed on {name}: {e}")
                    continue
                originals[name] = module
                _replace_module(model, name, replacement)
                replaced.add(name)
                count += 1
        if count:
            applied[pattern.name] = count

    if compile:
        import kernels.hip._torch_ops  # noqa: F401
        model = torch.compile(model, backend="inductor",
                              **({} if compile_mode == "default" else {"mode": compile_mode}))

    setattr(model, _STATE_ATTR, {
        "originals": originals,
        "applied": applied,
        "patterns": {p.name: p for p in patterns},
        "compiled": compile,
    })
    return model


def report(model: nn.Module) -> Dict[str, Any]:
    state = getattr(model, _STATE_ATTR, None)
    if state is None:
        return {"status": "not optimized", "patterns": {}}
    out: Dict[str, Any] = {"status": "optimized", "compiled": state["compiled"], "patterns": {}}
    for name, count in state["applied"].items():
        pattern = state["patterns"].get(name)
        out["patterns"][name] = {
            "modules_replaced": count,
            "op_speedup": f"{pattern.op_speedup:.1f}x" if pattern else "unknown",
        }
    return out


def restore(model: nn.Module) -> nn.Module:
    state = getattr(model, _STATE_ATTR, None)
    if state is None:
        return model
    for name, original in state["originals"].items():
        _replace_module(model, name, original)
    delattr(model, _STATE_ATTR)
    return model


def list_patterns() -> List[str]:
    return [p.name for p in ALL_PATTERNS]
