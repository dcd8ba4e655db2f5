"""ctypes wrapper around ``libak_oracle.so`` (C restatement of selective_scan_ref).

Test infrastructure only; see ``scan_ref.c``.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libak_oracle.so")
_lib = None


def available() -> bool:
    return os.path.exists(_LIB)


def _load():
    global _lib
    if _lib is None:
        _lib = ctypes.CDLL(_LIB)
        _lib.ak_oracle_selective_scan.argtypes = [ctypes.c_void_p] * 11 + [ctypes.c_int64] * 5 + [ctypes.c_int]
        _lib.ak_oracle_selective_scan.restype = None
    return _lib


def _f32(t: Optional[torch.Tensor]):
    return None if t is None else t.detach().to("cpu", torch.float32).contiguous()


def selective_scan(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                   initial_state=None):
    """Returns ``(out fp32 [b, d, l], last_state fp32 [b, d, n])``.

    An input-independent B or C (``[dim, n]``) is expanded to one group per
    channel (with the other one repeated to match), which is the same scan."""
    if B.dim() == 3:
        B = B.unsqueeze(1)
    if C.dim() == 3:
        C = C.unsqueeze(1)
    if B.dim() == 2 or C.dim() == 2:
        b_, d_, l_ = u.shape

        def per_channel(t):
            if t.dim() == 2:
                return t[None, :, :, None].expand(b_, d_, t.shape[1], l_)
            return t.repeat_interleave(d_ // t.shape[1], dim=1)

        B, C = per_channel(B), per_channel(C)
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    ngroups = B.shape[1]
    args = [_f32(t) for t in (u, delta, A, B, C, D, z, delta_bias, initial_state)]
    out = torch.empty(batch, dim, seqlen, dtype=torch.float32)
    last = torch.empty(batch, dim, dstate, dtype=torch.float32)
    ptr = lambda t: None if t is None else t.data_ptr()
    _load().ak_oracle_selective_scan(*[ptr(t) for t in args], out.data_ptr(), last.data_ptr(),
                                     batch, dim, seqlen, dstate, ngroups, int(bool(delta_softplus)))
    return out, last
