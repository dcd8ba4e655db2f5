"""Module-swap patterns for ``autokernel.optimize``.

Mirrors the reference's ``autokernel/_patterns.py``: a ``Pattern`` has a name,
a priority (higher applies first) and an informational ``op_speedup``;
``matches`` inspects a module, ``apply`` returns its replacement.

On gfx950 two patterns replace modules:

* ``fused_residual_rmsnorm`` (priority 100, reference :473-485): transformer
  blocks with (attention, attention_norm, feed_forward, ffn_norm)-style
  attributes. The replacement computes
  ``hidden, normed = fused_res_rmsnorm(attn_out, x, ffn_norm.weight)`` and
  returns ``hidden + feed_forward(normed)``. State-dict keys follow the
  reference replacement (``ffn_norm_weight``; reference :372).
* ``rmsnorm`` (priority 50, reference :508-529): RMSNorm-like modules.

The remaining reference patterns keep their names and priorities so that
``list_patterns()`` and include / exclude lists stay valid, but their kernels
(rotary, SwiGLU, Griffin scan) are not part of the gfx950 kernel set; they
never match.

The replacements always route through the autograd-registered custom ops
(``torch.ops.autokernel.*``) for fp16, bf16 and fp32 activations, with the
replaced norm module's own eps; the reference used the custom ops for fp16
only (PyTorch elsewhere) and a fixed eps of 1e-6.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, List, Optional

import torch
import torch.nn as nn


@dataclass
class Pattern:
    name: str
    priority: int
    op_speedup: float

    def matches(self, name: str, module: nn.Module, model: nn.Module) -> bool:
        raise NotImplementedError

    def apply(self, name: str, module: nn.Module, model: nn.Module) -> nn.Module:
        raise NotImplementedError


# Attribute-name aliases (ours, HuggingFace, and the reference's block families).
_BLOCK_ALIASES = [
    ("attention", "attention_norm", "feed_forward", "ffn_norm"),
    ("self_attn", "input_layernorm", "mlp", "post_attention_layernorm"),
    ("attn", "pre_norm", "ffn", "ffn_norm"),
    ("conv", "pre_norm", "ffn", "ffn_norm"),
]

_RMSNORM_CLASS_NAMES = {
    "RMSNorm", "LlamaRMSNorm", "MistralRMSNorm",
    "T5LayerNorm", "GemmaRMSNorm", "Qwen2RMSNorm",
}


def _find_block_attrs(module: nn.Module) -> Optional[tuple]:
    """(attn, attn_norm, ffn, ffn_norm) attribute names if ``module`` is a pre-norm block.

    Momentum blocks (``log_beta``) and modules flagged ``_skip_autokernel`` are
    rejected: their forward signatures differ.
    """
    if hasattr(module, "log_beta") or getattr(module, "_skip_autokernel", False):
        return None
    for attn, attn_norm, ffn, ffn_norm in _BLOCK_ALIASES:
        if (hasattr(module, attn) and hasattr(module, attn_norm) and hasattr(module, ffn)
                and hasattr(getattr(module, ffn_norm, None), "weight")):
            return attn, attn_norm, ffn, ffn_norm
    return None


def _autokernel_ops():
    import kernels.hip._torch_ops  # noqa: F401  (registers torch.ops.autokernel.*)
    return torch.ops.autokernel


def _norm_eps(norm: nn.Module) -> float:
    """The epsilon a norm module was built with: ``eps`` (torch.nn.RMSNorm and
    the reference's RMSNorm), ``variance_epsilon`` (HF Llama / Mistral / Qwen2 /
    T5), else the reference's fixed 1e-6. torch.nn.RMSNorm's ``eps=None``
    means the dtype's machine epsilon."""
    eps = getattr(norm, "eps", None)
    if eps is None and hasattr(norm, "variance_epsilon"):
        eps = norm.variance_epsilon
    if eps is None:
        w = getattr(norm, "weight", None)
        eps = torch.finfo(w.dtype).eps if isinstance(norm, getattr(nn, "RMSNorm", ())) and w is not None \
            else 1e-6
    return float(eps)


class _RMSNormReplacement(nn.Module):
    """RMSNorm through ``torch.ops.autokernel.rmsnorm`` with the module's own eps.

    HF's GemmaRMSNorm scales by ``1 + weight`` (its weight is stored as an
    offset from one); the replacement applies the same offset, so the swap
    keeps that module's output."""

    def __init__(self, original: nn.Module, kernel_fn: Callable):
        super().__init__()
        self.weight = original.weight
        self.eps = _norm_eps(original)
        self.weight_offset = 1.0 if type(original).__name__ == "GemmaRMSNorm" else 0.0
        self.kernel_fn = kernel_fn
        self._autograd_op = _autokernel_ops().rmsnorm

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        w = self.weight + self.weight_offset if self.weight_offset else self.weight
        out = self._autograd_op(x.reshape(-1, shape[-1]), w, float(self.eps))
        return out.view(shape)


class _FusedResidualRMSNormBlockReplacement(nn.Module):
    """Pre-norm block with the FFN-side residual add fused into the RMSNorm."""

    def __init__(self, original: nn.Module, kernel_fn_dual: Callable, attn_attr: str,
                 attn_norm_attr: str, ffn_attr: str, ffn_norm_attr: str):
        super().__init__()
        self.attention = getattr(original, attn_attr)
        self.attention_norm = getattr(original, attn_norm_attr)
        self.feed_forward = getattr(original, ffn_attr)
        ffn_norm = getattr(original, ffn_norm_attr)
        self.ffn_norm_weight = ffn_norm.weight
        self.eps = _norm_eps(ffn_norm)
        self.kernel_fn_dual = kernel_fn_dual
        self._autograd_dual = _autokernel_ops().fused_res_rmsnorm

    def forward(self, x: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
        attn_out = self.attention(self.attention_norm(x), freqs_cis)
        n = attn_out.shape[-1]
        hidden, normed = self._autograd_dual(attn_out.reshape(-1, n), x.reshape(-1, n),
                                             self.ffn_norm_weight, self.eps)
        hidden = hidden.view(attn_out.shape)
        normed = normed.view(attn_out.shape)
        return hidden + self.feed_forward(normed)


class FusedResidualRMSNormPattern(Pattern):
    def __init__(self):
        super().__init__("fused_residual_rmsnorm", priority=100, op_speedup=6.6)

    def matches(self, name, module, model):
        return _find_block_attrs(module) is not None

    def apply(self, name, module, model):
        from kernels.hip.fused_residual_add_rmsnorm import kernel_fn_dual
        return _FusedResidualRMSNormBlockReplacement(module, kernel_fn_dual, *_find_block_attrs(module))


class RMSNormPattern(Pattern):
    def __init__(self):
        super().__init__("rmsnorm", priority=50, op_speedup=3.3)

    def matches(self, name, module, model):
        if isinstance(module, torch.nn.RMSNorm) or getattr(module, "_native_norm", False):
            return False
        cls_name = type(module).__name__
        return (cls_name in _RMSNORM_CLASS_NAMES
                or (hasattr(module, "weight") and hasattr(module, "eps")
                    and not hasattr(module, "bias")
                    and cls_name.lower().endswith("norm")
                    and not isinstance(module, nn.LayerNorm)))

    def apply(self, name, module, model):
        from kernels.hip.rmsnorm import kernel_fn
        return _RMSNormReplacement(module, kernel_fn)


class _UnavailablePattern(Pattern):
    """A reference pattern whose kernel is outside the gfx950 kernel set: never matches."""

    def matches(self, name, module, model):
        return False

    def apply(self, name, module, model):
        raise RuntimeError(f"pattern {self.name!r} has no gfx950 kernel")


ALL_PATTERNS: List[Pattern] = [
    FusedResidualRMSNormPattern(),
    _UnavailablePattern("fused_griffin_block", priority=95, op_speedup=1.5),
    _UnavailablePattern("fused_qkv", priority=90, op_speedup=1.3),
    RMSNormPattern(),
    _UnavailablePattern("fused_silu_gate_mul", priority=45, op_speedup=1.6),
    _UnavailablePattern("silu_gate_mul", priority=40, op_speedup=1.6),
    _UnavailablePattern("rotary_embedding", priority=30, op_speedup=3.7),
]
