"""Helpers for the GPU parity tests."""

import sys

import pytest
import torch

gpu = pytest.mark.gpu


def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X GPU")


def say(*args):
    """Name the case before a GPU step (kept in the log if the step dies)."""
    print("[case]", *args, flush=True)
    sys.stdout.flush()


def ordered_bits(t: torch.Tensor) -> torch.Tensor:
    """Map fp16 / bf16 / fp32 values to integers whose order and spacing follow the
    floating-point grid (adjacent representable values differ by 1)."""
    if t.dtype in (torch.float16, torch.bfloat16):
        i = t.contiguous().view(torch.int16).to(torch.int64)
        return torch.where(i < 0, -32768 - i, i)
    if t.dtype == torch.float32:
        i = t.contiguous().view(torch.int32).to(torch.int64)
        return torch.where(i < 0, -(2 ** 31) - i, i)
    raise TypeError(t.dtype)


def max_ulp(a: torch.Tensor, b: torch.Tensor) -> int:
    """Largest distance in units in the last place between same-dtype tensors (NaN-free)."""
    assert a.dtype == b.dtype and a.shape == b.shape
    if a.numel() == 0:
        return 0
    return int((ordered_bits(a.cpu()) - ordered_bits(b.cpu())).abs().max())


def rel_err(a: torch.Tensor, b: torch.Tensor, floor: float = 0.0) -> float:
    a, b = a.double().cpu(), b.double().cpu()
    return float(((a - b).abs() / (b.abs() + floor)).max()) if a.numel() else 0.0
