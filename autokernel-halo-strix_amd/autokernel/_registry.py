"""Module swapping behind ``autokernel.optimize`` / ``report`` / ``restore``.

Public behaviour follows the reference ``autokernel/_registry.py:64-178``:
the same arguments, the same priority rule (a module that a higher-priority
pattern has swapped is not offered to a lower one), the same report
dictionary, and ``restore`` putting the original module objects back.

The implementation keeps one ``SwapRecord`` per optimized model: the modules
that were taken out (by qualified name), how many modules each pattern
swapped, and the pattern objects (for their ``op_speedup``). ``report`` is a
view of that record; ``restore`` replays it backwards and drops it.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, Iterable, List, Optional

import torch
import torch.nn as nn

from autokernel._patterns import ALL_PATTERNS, Pattern

# Attribute on the optimized model that holds its SwapRecord.
_STATE_ATTR = "_autokernel_state"


@dataclass
class SwapRecord:
    removed: Dict[str, nn.Module] = field(default_factory=dict)   # qualified name -> original
    counts: Dict[str, int] = field(default_factory=dict)          # pattern name -> modules swapped
    by_name: Dict[str, Pattern] = field(default_factory=dict)     # pattern name -> pattern
    compiled: bool = False


def _owner_and_leaf(root: nn.Module, qualified: str):
    *path, leaf = qualified.split(".")
    owner = root
    for part in path:
        owner = getattr(owner, part)
    return owner, leaf


def _set_submodule(root: nn.Module, qualified: str, module: nn.Module) -> None:
    owner, leaf = _owner_and_leaf(root, qualified)
    setattr(owner, leaf, module)


def _cast_keeping_complex(model: nn.Module, dtype: torch.dtype) -> nn.Module:
    """``model.to(dtype)``, except that complex buffers (rotary tables and the
    like) come back unchanged instead of being cast to a real dtype."""
    keep = {name: buf.clone() for name, buf in model.named_buffers() if buf.is_complex()}
    model = model.to(dtype=dtype)
    if keep:
        device = next(model.parameters()).device
        for name, buf in keep.items():
            owner, leaf = _owner_and_leaf(model, name)
            owner.register_buffer(leaf, buf.to(device), persistent=False)
    return model


def _chosen(include: Optional[Iterable[str]], exclude: Optional[Iterable[str]]) -> List[Pattern]:
    """Patterns named by include (all when None) minus those in exclude,
    highest priority first (ties keep their declaration order)."""
    wanted = None if include is None else set(include)
    unwanted = set() if exclude is None else set(exclude)
    chosen = [p for p in ALL_PATTERNS
              if (wanted is None or p.name in wanted) and p.name not in unwanted]
    return sorted(chosen, key=lambda p: -p.priority)


def _swap_all(model: nn.Module, patterns: List[Pattern], record: SwapRecord) -> None:
    for pattern in patterns:
        swapped = 0
        # a snapshot: the walk must not see the modules this loop puts in
        for name, module in list(model.named_modules()):
            if not name or name in record.removed:
                continue
            if not pattern.matches(name, module, model):
                continue
            try:
                new_module = pattern.apply(name, module, model)
            except Exception as err:  # the module stays as it was
                print(f"  autokernel: skipped {name}: pattern {pattern.name} raised {err}")
                continue
            record.removed[name] = module
            _set_submodule(model, name, new_module)
            swapped += 1
        if swapped:
            record.counts[pattern.name] = swapped


def optimize(model: nn.Module, dtype: torch.dtype = torch.float16, compile: bool = False,
             compile_mode: str = "default", include: Optional[List[str]] = None,
             exclude: Optional[List[str]] = None, training: bool = False) -> nn.Module:
    """Swap every module a selected pattern recognises for its gfx950
    replacement, in place, and return the model.

    For inference (``training=False``) the model is first cast to ``dtype``
    (complex buffers excepted) and put in eval mode; for training the
    parameter dtypes are left for autocast to handle and the mode is kept.
    The model is moved to the GPU when one is present. ``compile=True`` then
    wraps it in ``torch.compile``; the custom ops carry fake implementations,
    so they appear as opaque nodes in the traced graph.
    """
    if not training:
        model = _cast_keeping_complex(model, dtype)
    first = next(iter(model.parameters()), None)
    if torch.cuda.is_available() and first is not None and not first.is_cuda:
        model = model.cuda()
    if not training:
        model.eval()

    patterns = _chosen(include, exclude)
    record = SwapRecord(by_name={p.name: p for p in patterns}, compiled=bool(compile))
    _swap_all(model, patterns, record)

    if compile:
        import kernels.hip._torch_ops  # noqa: F401  (registers the custom ops)
        options = {} if compile_mode == "default" else {"mode": compile_mode}
        model = torch.compile(model, backend="inductor", **options)

    setattr(model, _STATE_ATTR, record)
    return model


def report(model: nn.Module) -> Dict[str, Any]:
    """What ``optimize`` did to ``model``: per pattern, the number of modules
    swapped and the pattern's quoted op speedup (formatted like ``"2.5x"``)."""
    record = getattr(model, _STATE_ATTR, None)
    if record is None:
        return {"status": "not optimized", "patterns": {}}
    per_pattern = {}
    for name, swapped in record.counts.items():
        pattern = record.by_name.get(name)
        speedup = "unknown" if pattern is None else f"{pattern.op_speedup:.1f}x"
        per_pattern[name] = {"modules_replaced": swapped, "op_speedup": speedup}
    return {"status": "optimized", "compiled": record.compiled, "patterns": per_pattern}


def restore(model: nn.Module) -> nn.Module:
    """Put back every original module ``optimize`` took out and forget the
    swap; a model that was never optimized is returned unchanged."""
    record = getattr(model, _STATE_ATTR, None)
    if record is None:
        return model
    for name in reversed(list(record.removed)):
        _set_submodule(model, name, record.removed[name])
    delattr(model, _STATE_ATTR)
    return model


def list_patterns() -> List[str]:
    """Names of every pattern ``optimize`` knows, in declaration order."""
    return [p.name for p in ALL_PATTERNS]
