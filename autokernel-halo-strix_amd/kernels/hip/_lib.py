"""Loader for the prebuilt gfx950 kernel library (``libautokernel_gfx950.so``).

Replaces the reference's JIT loader ``kernels/hip/_compile.py:210-369``
(``compile_hip`` -> ``torch.utils.cpp_extension.load_inline``): the kernels
are compiled ahead of time for gfx950 only (``csrc/Makefile``) and reached
through the C ABI declared in ``include/autokernel_mi355x.h``.

The library is opened after ``import torch`` so that its ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch has already loaded: kernels
launch on torch's current stream and use torch's device memory.

Every launcher here takes torch tensors, checks shapes and devices on the
host, and forwards raw pointers, element pitches and the current stream to
one ``extern "C"`` entry point. A non-zero return raises ``RuntimeError``
carrying ``ak_last_error()``. There is no CPU or PyTorch fallback: a missing
library or a non-GPU tensor raises.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading
from typing import Optional

import torch

LIB_NAME = "libautokernel_gfx950.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
CSRC_DIR = os.path.normpath(os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "..", "csrc"))

AK_DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
FLOAT_DTYPES = tuple(AK_DTYPE)
# complex64 (interleaved fp32 re, im): the selective scan's complex A
AK_DTYPE_C64 = 3

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_int = ctypes.c_int

# name -> argtypes (restype is int unless listed in _RESTYPES)
_SIGNATURES = {
    "ak_last_error": [],
    "ak_abi_version": [],
    "ak_target_arch": [],
    "ak_rmsnorm_fwd": [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _f32, _int, _c_void_p],
    "ak_fused_add_rmsnorm_fwd": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64,
                                 _i64, _i64, _i64, _i64, _f32, _int, _c_void_p],
    "ak_rmsnorm_bwd_workspace_bytes": [_i64, _i64],
    "ak_rmsnorm_bwd": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                       ctypes.c_size_t, _i64, _i64, _i64, _i64, _i64, _f32, _int, _c_void_p],
    "ak_fused_add_rmsnorm_bwd": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                 _c_void_p, ctypes.c_size_t, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _f32, _int, _c_void_p],
    "ak_fused_add_rmsnorm_bwd_noalloc": [_c_void_p] * 6 + [_i64] * 6 + [_f32, _int, _c_void_p],
    "ak_softmax_fwd": [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _int, _c_void_p],
    "ak_ce_fwd": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                  _i64, _i64, _i64, _i64, _f32, _i64, _f32, _f32, _f32, _c_void_p, _int, _c_void_p],
    "ak_ce_bwd_tiny": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                       _i64, _f32, _i64, _f32, _f32, _f32, _c_void_p, _int, _c_void_p],
    "ak_ce_count_valid": [_c_void_p, _i64, _i64, _c_void_p, _c_void_p],
    "ak_ce_mean": [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _f32, _c_void_p, _c_void_p,
                   _c_void_p],
    "ak_lmhead_ce_workspace_bytes": [_i64, _i64],
    "ak_lmhead_ce_fwd": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                         _c_void_p, ctypes.c_size_t, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _f32,
                         _int, _c_void_p],
    "ak_lmhead_ce_bwd": [_c_void_p] * 7 + [_i64] * 7 + [_f32, _f32, _int, _c_void_p],
    "ak_lmhead_ce_bwd_range": [_c_void_p] * 7 + [_i64] * 9 + [_f32, _f32, _int, _c_void_p],
    "ak_lmhead_grad_workspace_bytes": [_i64, _i64, _i64],
    "ak_lmhead_grad_hidden": [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64, _i64, _i64,
                              _int, _c_void_p, ctypes.c_size_t, _int, _c_void_p],
    "ak_lmhead_grad_weight": [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64, _i64, _i64,
                              _int, _c_void_p, ctypes.c_size_t, _int, _c_void_p],
    "ak_selective_scan_fwd": [_c_void_p] * 13 + [_i64] * 5 + [_i64] * 15 + [_int] * 6 + [_c_void_p],
    "ak_diag_scan_fwd": [_c_void_p] * 6 + [_i64] * 3 + [_c_void_p],
    "ak_diag_scan_bwd_workspace_bytes": [_i64, _i64],
    "ak_diag_scan_bwd": [_c_void_p] * 12 + [ctypes.c_size_t] + [_i64] * 3 + [_c_void_p],
    "ak_selective_scan_bwd_workspace_bytes": [_i64] * 5 + [_int],
    "ak_selective_scan_bwd": [_c_void_p] * 20 + [ctypes.c_size_t] + [_i64] * 5 + [_i64] * 15
    + [_int] * 6 + [_c_void_p],
}
_RESTYPES = {
    "ak_last_error": ctypes.c_char_p,
    "ak_target_arch": ctypes.c_char_p,
    "ak_lmhead_ce_workspace_bytes": ctypes.c_size_t,
    "ak_lmhead_grad_workspace_bytes": ctypes.c_size_t,
    "ak_rmsnorm_bwd_workspace_bytes": ctypes.c_size_t,
    "ak_diag_scan_bwd_workspace_bytes": ctypes.c_size_t,
    "ak_selective_scan_bwd_workspace_bytes": ctypes.c_size_t,
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


class HipExtensionMissing(RuntimeError):
    """The gfx950 kernel library has not been built."""


def lib_path() -> str:
    return os.environ.get("AUTOKERNEL_GFX950_LIB", LIB_PATH)


def load() -> ctypes.CDLL:
    """Open the kernel library (once) and declare every entry point."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = lib_path()
            if not os.path.exists(path):
                raise HipExtensionMissing(
                    f"{path} is missing: build it with `make -C {CSRC_DIR}` "
                    "or `python -c 'import __graft_entry__ as g; g.build()'`")
            handle = ctypes.CDLL(path)
            for name, argtypes in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.argtypes = argtypes
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = handle
    return _lib


def is_available() -> bool:
    return os.path.exists(lib_path())


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().ak_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# Per-call host overhead matters for small tensors (a 2048 x 768 RMSNorm runs
# in about 5 us on the GPU): the raw-stream query and the device check below
# avoid building a torch Stream object and entering a device guard per call.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
if _raw_stream is None:
    def _raw_stream(index: int) -> int:
        return torch.cuda.current_stream(index).cuda_stream
_NO_GUARD = contextlib.nullcontext()


def _stream(t: torch.Tensor) -> int:
    return _raw_stream(t.device.index)


def _on_device(t: torch.Tensor):
    """Device guard for launching on ``t``'s GPU (none when it is already current)."""
    if t.device.index == torch.cuda.current_device():
        return _NO_GUARD
    return torch.cuda.device(t.device)


def require_device(*tensors: Optional[torch.Tensor]) -> None:
    """Raise unless every given tensor lives on one GPU."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "autokernel gfx950 kernels need GPU tensors (got a tensor on "
                f"{t.device}); there is no CPU path")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return AK_DTYPE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected one of float32, float16, bfloat16")


def _rows_view(t: torch.Tensor, name: str) -> int:
    """Row pitch (elements) of a 2-D view whose last dim is contiguous.

    The pitch is passed on as it is, so rows that overlap (``stride(0) <
    cols``, e.g. an ``expand``-ed tensor with ``stride(0) == 0``) reach the
    C-ABI's pitch check and are rejected there; :func:`as_rows` copies such
    views first. A single row has no pitch and reports ``cols``."""
    shape = t.shape
    if len(shape) != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(shape)}")
    s0, s1 = t.stride()
    n0, n1 = shape
    if s1 != 1 and n1 > 1:
        raise ValueError(f"{name} must have a contiguous last dimension")
    return s0 if n0 > 1 else n1


def as_rows(t: torch.Tensor, cols: int) -> torch.Tensor:
    """``t`` as a ``[rows, cols]`` view the row kernels take: last dimension
    contiguous and rows that do not overlap (row pitch >= cols). Views that
    break either (a transposed last dim, an ``expand``-ed batch dim) are
    copied; everything else is passed through without a copy."""
    t2 = t.reshape(-1, cols)
    if (cols > 1 and t2.stride(-1) != 1) or (t2.shape[0] > 1 and t2.stride(0) < cols):
        t2 = t2.contiguous()
    return t2


# ---------------------------------------------------------------------------
# Launchers (tensor-level). Outputs are preallocated by the caller.
# ---------------------------------------------------------------------------

def rmsnorm(x: torch.Tensor, weight: torch.Tensor, y: torch.Tensor, eps: float) -> None:
    require_device(x, weight, y)
    rows, cols = x.shape
    with _on_device(x):
        rc = load().ak_rmsnorm_fwd(_ptr(x), _ptr(weight), _ptr(y), rows, cols,
                                   _rows_view(x, "x"), _rows_view(y, "y"), float(eps),
                                   dtype_code(x.dtype), _stream(x))
    _check(rc, "ak_rmsnorm_fwd")


def rmsnorm_contig(x: torch.Tensor, weight: torch.Tensor, y: torch.Tensor, cols: int,
                   eps: float) -> None:
    """RMSNorm of a contiguous ``x`` into a contiguous ``y`` of its shape and
    dtype, rows of ``cols`` elements, ``weight`` a contiguous ``[cols]`` of
    the same dtype. The caller has checked that all three are on one GPU;
    this launcher passes the dense pitch without building 2-D views (a view
    costs about 1 us of host time, the whole call about 4 us)."""
    n = x.numel()
    if n == 0:
        return
    dev = x.get_device()
    fn = (_lib or load()).ak_rmsnorm_fwd
    if dev == torch.cuda.current_device():
        rc = fn(x.data_ptr(), weight.data_ptr(), y.data_ptr(), n // cols, cols, cols, cols,
                eps, AK_DTYPE[x.dtype], _raw_stream(dev))
    else:
        with torch.cuda.device(dev):
            rc = fn(x.data_ptr(), weight.data_ptr(), y.data_ptr(), n // cols, cols, cols, cols,
                    eps, AK_DTYPE[x.dtype], _raw_stream(dev))
    if rc:
        _check(rc, "ak_rmsnorm_fwd")


def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                      new_residual: Optional[torch.Tensor], y: torch.Tensor, eps: float) -> None:
    require_device(x, residual, weight, new_residual, y)
    rows, cols = x.shape
    ld_nr = _rows_view(new_residual, "new_residual") if new_residual is not None else cols
    with _on_device(x):
        rc = load().ak_fused_add_rmsnorm_fwd(
            _ptr(x), _ptr(residual), _ptr(weight), _ptr(new_residual), _ptr(y), rows, cols,
            _rows_view(x, "x"), _rows_view(residual, "residual"), ld_nr, _rows_view(y, "y"),
            float(eps), dtype_code(x.dtype), _stream(x))
    _check(rc, "ak_fused_add_rmsnorm_fwd")


def rmsnorm_bwd_workspace_bytes(rows: int, cols: int) -> int:
    return int(load().ak_rmsnorm_bwd_workspace_bytes(rows, cols))


def rmsnorm_bwd(x: torch.Tensor, weight: torch.Tensor, grad_out: torch.Tensor,
                grad_x: torch.Tensor, grad_weight: Optional[torch.Tensor],
                workspace: Optional[torch.Tensor], eps: float) -> None:
    """RMSNorm backward over 2-D ``[rows, cols]`` views; grad_weight fp32 ``[cols]``."""
    require_device(x, weight, grad_out, grad_x, grad_weight, workspace)
    rows, cols = x.shape
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    with _on_device(x):
        rc = load().ak_rmsnorm_bwd(
            _ptr(x), _ptr(weight), _ptr(grad_out), _ptr(grad_x), _ptr(grad_weight),
            _ptr(workspace), ws_bytes, rows, cols, _rows_view(x, "x"),
            _rows_view(grad_out, "grad_out"), _rows_view(grad_x, "grad_x"), float(eps),
            dtype_code(x.dtype), _stream(x))
    _check(rc, "ak_rmsnorm_bwd")


def fused_add_rmsnorm_bwd(hidden: torch.Tensor, weight: torch.Tensor,
                          grad_hidden: Optional[torch.Tensor], grad_normed: torch.Tensor,
                          grad_x: torch.Tensor, grad_weight: Optional[torch.Tensor],
                          workspace: Optional[torch.Tensor], eps: float) -> None:
    """Fused residual + RMSNorm backward over 2-D views; grad_hidden may be None."""
    require_device(hidden, weight, grad_hidden, grad_normed, grad_x, grad_weight, workspace)
    rows, cols = hidden.shape
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    ld_gh = _rows_view(grad_hidden, "grad_hidden") if grad_hidden is not None else cols
    with _on_device(hidden):
        rc = load().ak_fused_add_rmsnorm_bwd(
            _ptr(hidden), _ptr(weight), _ptr(grad_hidden), _ptr(grad_normed), _ptr(grad_x),
            _ptr(grad_weight), _ptr(workspace), ws_bytes, rows, cols,
            _rows_view(hidden, "hidden"), ld_gh, _rows_view(grad_normed, "grad_normed"),
            _rows_view(grad_x, "grad_x"), float(eps), dtype_code(hidden.dtype), _stream(hidden))
    _check(rc, "ak_fused_add_rmsnorm_bwd")


# Bytes of one stream's slot of the fixed scratch behind
# ak_fused_add_rmsnorm_bwd_noalloc (four slots per GPU, one per calling stream).
NOALLOC_SCRATCH_BYTES = 16 << 20
NOALLOC_STREAM_SLOTS = 4


def fused_add_rmsnorm_bwd_noalloc(hidden: torch.Tensor, weight: torch.Tensor,
                                  grad_hidden: Optional[torch.Tensor], grad_normed: torch.Tensor,
                                  grad_x: torch.Tensor, grad_weight: Optional[torch.Tensor],
                                  eps: float) -> None:
    """:func:`fused_add_rmsnorm_bwd` through the entry point that allocates
    nothing (a slot of the library's fixed scratch, owned by the current
    stream, holds the partial weight-gradient rows); shapes beyond a slot, and
    a fifth calling stream on one GPU, raise."""
    require_device(hidden, weight, grad_hidden, grad_normed, grad_x, grad_weight)
    rows, cols = hidden.shape
    ld_gh = _rows_view(grad_hidden, "grad_hidden") if grad_hidden is not None else cols
    with _on_device(hidden):
        rc = load().ak_fused_add_rmsnorm_bwd_noalloc(
            _ptr(hidden), _ptr(weight), _ptr(grad_hidden), _ptr(grad_normed), _ptr(grad_x),
            _ptr(grad_weight), rows, cols, _rows_view(hidden, "hidden"), ld_gh,
            _rows_view(grad_normed, "grad_normed"), _rows_view(grad_x, "grad_x"), float(eps),
            dtype_code(hidden.dtype), _stream(hidden))
    _check(rc, "ak_fused_add_rmsnorm_bwd_noalloc")


def softmax(x: torch.Tensor, y: torch.Tensor) -> None:
    require_device(x, y)
    rows, cols = x.shape
    with _on_device(x):
        rc = load().ak_softmax_fwd(_ptr(x), _ptr(y), rows, cols, _rows_view(x, "x"),
                                   _rows_view(y, "y"), dtype_code(x.dtype), _stream(x))
    _check(rc, "ak_softmax_fwd")


def ce_fwd(logits: torch.Tensor, targets: torch.Tensor, losses: torch.Tensor, lse: torch.Tensor,
           row_max: Optional[torch.Tensor], row_sum: Optional[torch.Tensor],
           grad: Optional[torch.Tensor], softcap: float, ignore_index: int,
           label_smoothing: float, scale_grad: float,
           scale_dev: Optional[torch.Tensor] = None, z_loss_weight: float = 0.0) -> None:
    """Per-row CE over ``logits [rows, vocab]``; the gradient (when ``grad`` is
    given, including the z-loss term) is scaled by ``scale_grad`` times the
    device value ``scale_dev[0]``."""
    require_device(logits, targets, losses, lse, row_max, row_sum, grad, scale_dev)
    rows, vocab = logits.shape
    ld_g = _rows_view(grad, "grad") if grad is not None else vocab
    with _on_device(logits):
        rc = load().ak_ce_fwd(_ptr(logits), _ptr(targets), _ptr(losses), _ptr(lse), _ptr(row_max),
                              _ptr(row_sum), _ptr(grad), rows, vocab, _rows_view(logits, "logits"),
                              ld_g, float(softcap), int(ignore_index), float(label_smoothing),
                              float(scale_grad), float(z_loss_weight), _ptr(scale_dev),
                              dtype_code(logits.dtype),
                              _stream(logits))
    _check(rc, "ak_ce_fwd")


def ce_bwd_tiny(logits: torch.Tensor, targets: torch.Tensor, row_max: torch.Tensor,
                row_sum: torch.Tensor, grad: torch.Tensor, softcap: float, ignore_index: int,
                label_smoothing: float, scale_grad: float, z_loss_weight: float = 0.0,
                scale_dev: Optional[torch.Tensor] = None) -> None:
    require_device(logits, targets, row_max, row_sum, grad, scale_dev)
    rows, vocab = logits.shape
    with _on_device(logits):
        rc = load().ak_ce_bwd_tiny(_ptr(logits), _ptr(targets), _ptr(row_max), _ptr(row_sum),
                                   _ptr(grad), rows, vocab, _rows_view(logits, "logits"),
                                   _rows_view(grad, "grad"), float(softcap), int(ignore_index),
                                   float(label_smoothing), float(scale_grad),
                                   float(z_loss_weight), _ptr(scale_dev),
                                   dtype_code(logits.dtype), _stream(logits))
    _check(rc, "ak_ce_bwd_tiny")


def ce_count_valid(targets: torch.Tensor, ignore_index: int) -> torch.Tensor:
    """fp32 device tensor ``[max(1, #counted rows), 1 / that]``."""
    require_device(targets)
    denom = torch.empty(2, dtype=torch.float32, device=targets.device)
    with _on_device(targets):
        rc = load().ak_ce_count_valid(_ptr(targets), targets.numel(), int(ignore_index),
                                      _ptr(denom), _stream(targets))
    _check(rc, "ak_ce_count_valid")
    return denom


def ce_mean(losses: torch.Tensor, lse: Optional[torch.Tensor], targets: torch.Tensor,
            ignore_index: int, z_loss_weight: float = 0.0,
            n_valid: Optional[torch.Tensor] = None) -> torch.Tensor:
    """0-d fp32 device tensor: the mean (+ z-loss) over counted rows."""
    require_device(losses, lse, targets, n_valid)
    loss = torch.empty((), dtype=torch.float32, device=losses.device)
    with _on_device(losses):
        rc = load().ak_ce_mean(_ptr(losses), _ptr(lse), _ptr(targets), targets.numel(),
                               int(ignore_index), float(z_loss_weight), _ptr(loss),
                               _ptr(n_valid), _stream(losses))
    _check(rc, "ak_ce_mean")
    return loss


def lmhead_ce_workspace_bytes(n_rows: int, vocab: int) -> int:
    return int(load().ak_lmhead_ce_workspace_bytes(n_rows, vocab))


def lmhead_ce(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
              loss: torch.Tensor, lse: torch.Tensor, losses: Optional[torch.Tensor],
              n_valid: Optional[torch.Tensor], workspace: torch.Tensor, ignore_index: int,
              softcap: float = 0.0, label_smoothing: float = 0.0) -> None:
    require_device(hidden, weight, targets, loss, lse, losses, n_valid, workspace)
    n_rows, d = hidden.shape
    vocab = weight.shape[0]
    with _on_device(hidden):
        rc = load().ak_lmhead_ce_fwd(
            _ptr(hidden), _ptr(weight), _ptr(targets), _ptr(loss), _ptr(lse), _ptr(losses),
            _ptr(n_valid), _ptr(workspace), workspace.numel() * workspace.element_size(),
            n_rows, vocab, d, _rows_view(hidden, "hidden"), _rows_view(weight, "weight"),
            int(ignore_index), float(softcap), float(label_smoothing), dtype_code(hidden.dtype),
            _stream(hidden))
    _check(rc, "ak_lmhead_ce_fwd")


def lmhead_ce_bwd(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                  lse: torch.Tensor, grad_loss: torch.Tensor, denom: torch.Tensor,
                  grad_logits: torch.Tensor, ignore_index: int, softcap: float = 0.0,
                  label_smoothing: float = 0.0) -> None:
    """dL/dlogits of the mean CE into ``grad_logits`` ``[n_rows, vocab]`` (row pitch a
    multiple of 4); ``grad_loss`` and ``denom`` are 1-element fp32 device tensors."""
    require_device(hidden, weight, targets, lse, grad_loss, denom, grad_logits)
    n_rows, d = hidden.shape
    vocab = weight.shape[0]
    with _on_device(hidden):
        rc = load().ak_lmhead_ce_bwd(
            _ptr(hidden), _ptr(weight), _ptr(targets), _ptr(lse), _ptr(grad_loss), _ptr(denom),
            _ptr(grad_logits), _rows_view(grad_logits, "grad_logits"), n_rows, vocab, d,
            _rows_view(hidden, "hidden"), _rows_view(weight, "weight"), int(ignore_index),
            float(softcap), float(label_smoothing), dtype_code(hidden.dtype), _stream(hidden))
    _check(rc, "ak_lmhead_ce_bwd")


def lmhead_ce_bwd_range(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                        lse: torch.Tensor, grad_loss: torch.Tensor, denom: torch.Tensor,
                        grad_logits: torch.Tensor, v_begin: int, ignore_index: int,
                        softcap: float = 0.0, label_smoothing: float = 0.0) -> None:
    """:func:`lmhead_ce_bwd` for the vocab columns ``[v_begin, v_begin +
    grad_logits.shape[1])`` of the full ``weight``'s vocabulary."""
    require_device(hidden, weight, targets, lse, grad_loss, denom, grad_logits)
    n_rows, d = hidden.shape
    vocab = weight.shape[0]
    with _on_device(hidden):
        rc = load().ak_lmhead_ce_bwd_range(
            _ptr(hidden), _ptr(weight), _ptr(targets), _ptr(lse), _ptr(grad_loss), _ptr(denom),
            _ptr(grad_logits), _rows_view(grad_logits, "grad_logits"), n_rows, vocab,
            int(v_begin), grad_logits.shape[1], d, _rows_view(hidden, "hidden"),
            _rows_view(weight, "weight"), int(ignore_index), float(softcap),
            float(label_smoothing), dtype_code(hidden.dtype), _stream(hidden))
    _check(rc, "ak_lmhead_ce_bwd_range")


# out_mode of the lm-head gradient GEMMs
GEMM_OUT_DTYPE = 0     # store in the operands' dtype
GEMM_OUT_F32 = 1       # store fp32
GEMM_OUT_F32_ADD = 2   # add into an fp32 output


def lmhead_grad_workspace_bytes(n_rows: int, vocab: int, d: int) -> int:
    return int(load().ak_lmhead_grad_workspace_bytes(n_rows, vocab, d))


def _grad_gemm(entry: str, grad_logits: torch.Tensor, operand: torch.Tensor,
               out: torch.Tensor, out_mode: int, workspace: Optional[torch.Tensor]) -> None:
    require_device(grad_logits, operand, out, workspace)
    if grad_logits.dim() != 2 or operand.dim() != 2 or out.dim() != 2:
        raise ValueError(f"{entry}: grad_logits, operand and out must be 2-D")
    n_rows, vocab = grad_logits.shape
    d = operand.shape[1]
    if operand.dtype != grad_logits.dtype:
        raise ValueError(f"{entry}: operand dtype {operand.dtype} != grad_logits dtype {grad_logits.dtype}")
    want_out = grad_logits.dtype if out_mode == GEMM_OUT_DTYPE else torch.float32
    if out_mode not in (GEMM_OUT_DTYPE, GEMM_OUT_F32, GEMM_OUT_F32_ADD) or out.dtype != want_out:
        raise ValueError(f"{entry}: out_mode {out_mode} needs a {want_out} output, got {out.dtype}")
    # grad_hidden: operand [vocab, d], out [n_rows, d]; grad_weight: operand [n_rows, d], out [vocab, d]
    rows_op, rows_out = (vocab, n_rows) if entry == "ak_lmhead_grad_hidden" else (n_rows, vocab)
    if operand.shape[0] != rows_op or tuple(out.shape) != (rows_out, d):
        raise ValueError(f"{entry}: shapes grad_logits {tuple(grad_logits.shape)}, operand "
                         f"{tuple(operand.shape)}, out {tuple(out.shape)} do not fit")
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    with _on_device(grad_logits):
        rc = getattr(load(), entry)(
            _ptr(grad_logits), grad_logits.stride(0), _ptr(operand), _rows_view(operand, "operand"),
            _ptr(out), _rows_view(out, "out"), n_rows, vocab, d, int(out_mode), _ptr(workspace),
            ws_bytes, dtype_code(grad_logits.dtype), _stream(grad_logits))
    _check(rc, entry)


def _zero_k_padding(grad_logits: torch.Tensor) -> None:
    """Zero columns ``[vocab, vocab rounded up to 64)`` behind a ``[n_rows,
    vocab]`` dlogits view. ak_lmhead_grad_hidden reads whole 64-column K
    blocks and multiplies the padding by weight rows that load as zeros, so
    any finite padding adds nothing, but a NaN or Inf left in fresh memory
    would turn 0 x NaN into NaN. Also checks that the storage holds
    ``n_rows`` whole row pitches, the extent the kernel reads."""
    n_rows, vocab = grad_logits.shape
    pitch = grad_logits.stride(0)
    vpad = -(-vocab // 64) * 64
    if pitch < vpad:
        raise ValueError(f"grad_logits row pitch {pitch} must cover vocab rounded up to 64 ({vpad})")
    size = grad_logits.untyped_storage().nbytes() // grad_logits.element_size()
    if grad_logits.storage_offset() + n_rows * pitch > size:
        raise ValueError("grad_logits storage must hold n_rows whole row pitches")
    if vpad > vocab and n_rows:
        torch.as_strided(grad_logits, (n_rows, vpad - vocab), (pitch, 1),
                         grad_logits.storage_offset() + vocab).zero_()


def lmhead_grad_hidden(grad_logits: torch.Tensor, weight: torch.Tensor, out: torch.Tensor,
                       out_mode: int, workspace: Optional[torch.Tensor]) -> None:
    """out (=, or += with GEMM_OUT_F32_ADD) grad_logits @ weight.

    ``grad_logits`` is a ``[n_rows, vocab]`` view whose row pitch covers
    vocab rounded up to 64 (the padding columns are zeroed here, and the
    storage must hold ``n_rows`` whole pitches); ``weight`` is ``[vocab, d]``;
    ``out`` is ``[n_rows, d]``."""
    if grad_logits.stride(1) != 1:
        raise ValueError("grad_logits must have a contiguous last dimension")
    _zero_k_padding(grad_logits)
    _grad_gemm("ak_lmhead_grad_hidden", grad_logits, weight, out, out_mode, workspace)


def lmhead_grad_weight(grad_logits: torch.Tensor, hidden: torch.Tensor, out: torch.Tensor,
                       out_mode: int, workspace: Optional[torch.Tensor]) -> None:
    """out (=, or += with GEMM_OUT_F32_ADD) grad_logits^T @ hidden; ``out``
    is ``[vocab, d]``, the other operands as in :func:`lmhead_grad_hidden`."""
    if grad_logits.stride(1) != 1:
        raise ValueError("grad_logits must have a contiguous last dimension")
    _grad_gemm("ak_lmhead_grad_weight", grad_logits, hidden, out, out_mode, workspace)


# bc_flags of the selective-scan entry points: B / C input-independent ([dim, dstate] fp32)
SCAN_B_CONST = 1
SCAN_C_CONST = 2
SCAN_A_COMPLEX = 4  # workspace query only


def _scan_bc(B: torch.Tensor, C: torch.Tensor):
    """(bc_flags, B strides, C strides, ngroups, element-type code of the variable
    B / C) for B / C that are either variable ``[batch, ngroups, dstate, seqlen]``
    or input-independent ``[dim, dstate]`` fp32."""
    flags = 0
    if B.dim() == 2:
        flags |= SCAN_B_CONST
        bs = (0, B.stride(0), B.stride(1))
    else:
        bs = (B.stride(0), B.stride(1), B.stride(2))
    if C.dim() == 2:
        flags |= SCAN_C_CONST
        cs = (0, C.stride(0), C.stride(1))
    else:
        cs = (C.stride(0), C.stride(1), C.stride(2))
    var = [t for t in (B, C) if t.dim() == 4]
    ngroups = var[0].shape[1] if var else 1
    bc_dtype = dtype_code(var[0].dtype) if var else AK_DTYPE[torch.float32]
    return flags, bs, cs, ngroups, bc_dtype


def _a_code(A: torch.Tensor) -> int:
    return AK_DTYPE_C64 if A.dtype == torch.complex64 else dtype_code(A.dtype)


def selective_scan(u, delta, A, B, C, D, z, delta_bias, out, last_state, delta_softplus: bool,
                   out_prez=None, chunk_states=None, checkpoints=None) -> None:
    """Mamba-1 forward. u/delta/z/out [b, d, l]; B/C [b, g, n, l] or input-independent
    [d, n] fp32; A [d, n] fp32; optional out_prez (pre-gate output, strides of out),
    chunk_states [b, d, ceil(l/2048), n, 2] and checkpoints [b, ceil(l/16), d, n]
    (the states the backward restarts from). With a complex64 A: a variable B/C is
    real [b, g, n, 2l] of (re, im) pairs, a constant one complex64 [d, n], and
    last_state / chunk_states / checkpoints are complex64."""
    require_device(u, delta, A, B, C, D, z, delta_bias, out, last_state, out_prez, chunk_states,
                   checkpoints)
    if out_prez is not None and out_prez.stride() != out.stride():
        raise ValueError("out_prez must have out's strides")
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    flags, bs, cs, ngroups, bc_dtype = _scan_bc(B, C)
    zs = (z.stride(0), z.stride(1)) if z is not None else (0, 0)
    with _on_device(u):
        rc = load().ak_selective_scan_fwd(
            _ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C), _ptr(D), _ptr(z), _ptr(delta_bias),
            _ptr(out), _ptr(last_state), _ptr(out_prez), _ptr(chunk_states), _ptr(checkpoints),
            batch, dim, seqlen, dstate, ngroups,
            u.stride(0), u.stride(1), delta.stride(0), delta.stride(1), A.stride(0),
            *bs, *cs, zs[0], zs[1], out.stride(0), out.stride(1),
            int(bool(delta_softplus)), flags, dtype_code(u.dtype), dtype_code(delta.dtype),
            bc_dtype, _a_code(A), _stream(u))
    _check(rc, "ak_selective_scan_fwd")


def selective_scan_bwd(u, delta, A, B, C, D, z, delta_bias, dout, du, ddelta, dA, dB, dC, dD, dz,
                       ddelta_bias, delta_softplus: bool, checkpoints=None, out_prez=None) -> None:
    """Mamba-1 backward. u/delta/z/dout [b, d, l] (last dim contiguous); B/C
    [b, g, n, l] or input-independent [d, n] fp32; A [d, n]; outputs du/ddelta/dz
    contiguous [b, d, l], dB/dC contiguous in B's / C's layout (a variable one in
    its dtype, an input-independent one fp32), dA [d, n] / dD [d] / ddelta_bias [d]
    fp32. With the forward's ``checkpoints`` (and, with z, its contiguous
    ``out_prez``) the states are not recomputed. With a complex64 A, dA and an
    input-independent dB / dC are complex64 (layouts as in :func:`selective_scan`)."""
    require_device(u, delta, A, B, C, D, z, delta_bias, dout, du, ddelta, dA, dB, dC, dD, dz,
                   ddelta_bias, checkpoints, out_prez)
    if out_prez is not None and not out_prez.is_contiguous():
        raise ValueError("out_prez must be contiguous")
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    flags, bs, cs, ngroups, bc_dtype = _scan_bc(B, C)
    zs = (z.stride(0), z.stride(1)) if z is not None else (0, 0)
    lib = load()
    wflags = flags | (SCAN_A_COMPLEX if A.is_complex() else 0)
    ws = torch.empty(int(lib.ak_selective_scan_bwd_workspace_bytes(batch, dim, seqlen, dstate,
                                                                   ngroups, wflags)),
                     dtype=torch.uint8, device=u.device)
    with _on_device(u):
        rc = lib.ak_selective_scan_bwd(
            _ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C), _ptr(D), _ptr(z), _ptr(delta_bias),
            _ptr(dout), _ptr(du), _ptr(ddelta), _ptr(dA), _ptr(dB), _ptr(dC), _ptr(dD), _ptr(dz),
            _ptr(ddelta_bias), _ptr(checkpoints), _ptr(out_prez), _ptr(ws), ws.numel(),
            batch, dim, seqlen, dstate, ngroups,
            u.stride(0), u.stride(1), delta.stride(0), delta.stride(1), A.stride(0),
            *bs, *cs, zs[0], zs[1], dout.stride(0), dout.stride(1),
            int(bool(delta_softplus)), flags, dtype_code(u.dtype), dtype_code(delta.dtype),
            bc_dtype, _a_code(A), _stream(u))
    _check(rc, "ak_selective_scan_bwd")


def diag_scan(dA, dBx, C, D, x, y) -> None:
    require_device(dA, dBx, C, D, x, y)
    batch, seqlen, d_inner = dA.shape
    with _on_device(dA):
        rc = load().ak_diag_scan_fwd(_ptr(dA), _ptr(dBx), _ptr(C), _ptr(D), _ptr(x), _ptr(y),
                                     batch, seqlen, d_inner, _stream(dA))
    _check(rc, "ak_diag_scan_fwd")


def diag_scan_bwd(dA, dBx, C, D, x, grad_y, grad_dA, grad_dBx, grad_C, grad_D, grad_x) -> None:
    """Backward of :func:`diag_scan`; all fp32, contiguous ``[batch, seq, d_inner]``."""
    require_device(dA, dBx, C, D, x, grad_y, grad_dA, grad_dBx, grad_C, grad_D, grad_x)
    batch, seqlen, d_inner = dA.shape
    lib = load()
    ws = torch.empty(int(lib.ak_diag_scan_bwd_workspace_bytes(batch, d_inner)), dtype=torch.uint8,
                     device=dA.device)
    with _on_device(dA):
        rc = lib.ak_diag_scan_bwd(_ptr(dA), _ptr(dBx), _ptr(C), _ptr(D), _ptr(x), _ptr(grad_y),
                                  _ptr(grad_dA), _ptr(grad_dBx), _ptr(grad_C), _ptr(grad_D),
                                  _ptr(grad_x), _ptr(ws), ws.numel(), batch, seqlen, d_inner,
                                  _stream(dA))
    _check(rc, "ak_diag_scan_bwd")
