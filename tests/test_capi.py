"""The C-ABI library loads and exports every entry point the header declares (CPU tier).

No compute entry point is called here (no GPU in this tier); only argument
validation paths that return before any HIP call.
"""

import ctypes
import os
import re

import pytest

from kernels.hip import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "autokernel_mi355x.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\*?\s+(ak_[a-z0-9_]+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.is_available():
        pytest.skip("libautokernel_gfx950.so not built")
    return _lib.load()


def test_header_declares_the_loader_signatures():
    assert _declared() == sorted(_lib.EXPORTED_SYMBOLS)


def test_every_declared_symbol_is_exported(lib):
    for name in _declared():
        assert hasattr(lib, name), name


def test_version_and_arch(lib):
    assert lib.ak_abi_version() == 2
    assert lib.ak_target_arch() == b"gfx950"


def test_workspace_query(lib):
    ws = _lib.lmhead_ce_workspace_bytes(8192, 50304)
    n_vt = (50304 + 255) // 256
    # (max, sum) partials + per-row losses + label smoothing's per-partial logit sums
    assert ws >= n_vt * 8192 * 8 + 8192 * 4 + 2 * n_vt * 8192 * 4
    assert ws % 256 == 0
    assert _lib.lmhead_ce_workspace_bytes(0, 10) == 0


def test_argument_errors_return_codes(lib):
    # unsupported dtype code, rejected before any HIP call
    rc = lib.ak_rmsnorm_fwd(None, None, None, 4, 8, 8, 8, 1e-6, 7, None)
    assert rc == -2 and b"dtype" in lib.ak_last_error()
    rc = lib.ak_softmax_fwd(None, None, 4, 8, 4, 8, 0, None)   # pitch < cols
    assert rc == -1 and b"pitch" in lib.ak_last_error()
    rc = lib.ak_lmhead_ce_fwd(None, None, None, None, None, None, None, None, 0, 8, 16, 100, 100, 100, -100, 0.0, 0.0, 2, None)
    assert rc == -2 and b"multiple" in lib.ak_last_error()
    rc = lib.ak_lmhead_ce_fwd(None, None, None, None, None, None, None, None, 0, 8, 16, 64, 64, 64, -100, 0.0, 0.0, 0, None)
    assert rc == -2  # fp32 is not a matrix-core input type here
    rc = lib.ak_lmhead_ce_fwd(None, None, None, None, None, None, None, None, 0, 8, 16, 64, 64, 64, -100, -1.0, 0.0, 2, None)
    assert rc == -1 and b"softcap" in lib.ak_last_error()
    rc = lib.ak_lmhead_ce_bwd(*([None] * 7), 16, 8, 16, 64, 64, 64, -100, float("nan"), 0.0, 2, None)
    assert rc == -1 and b"softcap" in lib.ak_last_error()
    for ls in (-0.1, 1.5, float("nan")):
        rc = lib.ak_lmhead_ce_fwd(*([None] * 8), 0, 8, 16, 64, 64, 64, -100, 0.0, ls, 2, None)
        assert rc == -1 and b"label_smoothing" in lib.ak_last_error()
        rc = lib.ak_lmhead_ce_bwd(*([None] * 7), 16, 8, 16, 64, 64, 64, -100, 0.0, ls, 2, None)
        assert rc == -1 and b"label_smoothing" in lib.ak_last_error()
    # vocab ranges: inside [0, vocab), grad_logits pitch >= the range's width
    for v_begin, v_count in ((-1, 8), (0, 0), (60, 8), (0, 65)):
        rc = lib.ak_lmhead_ce_bwd_range(*([None] * 7), 16, 8, 64, v_begin, v_count, 64, 64, 64, -100,
                                        0.0, 0.0, 2, None)
        assert rc == -1 and b"vocab range" in lib.ak_last_error()
    rc = lib.ak_lmhead_ce_bwd_range(*([None] * 7), 8, 8, 64, 16, 32, 64, 64, 64, -100, 0.0, 0.0, 2, None)
    assert rc == -1 and b"pitch" in lib.ak_last_error()
    rc = _lib.load().ak_selective_scan_fwd(*([None] * 13), 2, 4, 16, 300, 1, *([0] * 15), 0, 0, 2, 0,
                                           2, 0, None)
    assert rc == -2 and b"dstate" in lib.ak_last_error()
    # zero-size work is a no-op success
    assert lib.ak_rmsnorm_fwd(None, None, None, 0, 8, 8, 8, 1e-6, 0, None) == 0


def test_lmhead_grad_gemm_workspace_and_argument_errors(lib):
    """The gradient GEMMs' workspace holds the fp32 partial tiles of the
    K-split work; with no GPU the CU count defaults to MI355X's 256. At the C4
    shape grad_hidden's 96 tiles run 8 K ranges each (the larger of the two
    GEMMs' needs)."""
    assert _lib.lmhead_grad_workspace_bytes(8192, 50304, 768) == 96 * 8 * 256 * 256 * 4
    assert _lib.lmhead_grad_workspace_bytes(0, 10, 64) == 0
    f = lib.ak_lmhead_grad_hidden
    # (grad_logits, ld_gl, operand, ld_op, out, ld_out, n_rows, vocab, d, out_mode, ws, ws_bytes, dtype, stream)
    rc = f(None, 1024, None, 64, None, 64, 8, 1000, 64, 0, None, 0, 0, None)
    assert rc == -2 and b"dtype" in lib.ak_last_error()
    rc = f(None, 1024, None, 96, None, 96, 8, 1000, 96, 0, None, 0, 2, None)
    assert rc == -2 and b"multiple of 64" in lib.ak_last_error()
    rc = f(None, 1000, None, 64, None, 64, 8, 1000, 64, 0, None, 0, 2, None)   # pitch < round_up(vocab, 64)
    assert rc == -1 and b"pitch" in lib.ak_last_error()
    rc = f(None, 1024, None, 64, None, 64, 8, 1000, 64, 3, None, 0, 2, None)
    assert rc == -1 and b"out_mode" in lib.ak_last_error()
    rc = lib.ak_lmhead_grad_weight(None, 1024, None, 64, None, 64, 8, 1000, 64, 0, None, 0, 2, None)
    assert rc == -1 and b"null" in lib.ak_last_error()


def test_selective_scan_bwd_workspace_and_argument_errors(lib):
    """Workspace query of the Mamba-1 backward (saved states every 16 steps,
    per-tile dB / dC partials, per-batch dA / dD / ddelta_bias partials, each
    256-byte aligned) and its argument checks, all rejected before any HIP
    call."""
    a256 = lambda v: (v + 255) // 256 * 256
    b, d, l, n, g = 2, 40, 100, 16, 2
    tiles = (d // g + 15) // 16
    want = (a256(b * ((l + 15) // 16) * d * n * 4) + 2 * a256(tiles * b * g * n * l * 4)
            + a256(b * d * n * 4) + 2 * a256(b * d * 4))
    assert lib.ak_selective_scan_bwd_workspace_bytes(b, d, l, n, g, 0) == want
    assert lib.ak_selective_scan_bwd_workspace_bytes(0, d, l, n, g, 0) == 0
    assert lib.ak_selective_scan_bwd_workspace_bytes(b, 41, l, n, g, 0) == 0  # dim % ngroups
    fn = _lib.load().ak_selective_scan_bwd
    strides = [0] * 15
    rc = fn(*([None] * 19), None, 0, 2, 4, 16, 300, 1, *strides, 0, 0, 2, 0, 2, 0, None)
    assert rc == -2 and b"dstate" in lib.ak_last_error()
    fake = 4096  # never dereferenced: every check below fails first
    ptrs = [fake] * 17 + [None, None]  # no saved checkpoints / out_prez
    ptrs[14] = None  # dD missing while D is given
    rc = fn(*ptrs, None, 0, 2, 4, 16, 8, 1, *strides, 0, 0, 2, 0, 2, 0, None)
    assert rc == -1 and b"dD" in lib.ak_last_error()
    rc = fn(*([fake] * 17), fake, None, fake, 1 << 30, 2, 4, 64, 8, 1, *strides, 0, 0, 2, 0, 2, 0, None)
    assert rc == -1 and b"out_prez" in lib.ak_last_error()  # checkpoints and z without out_prez
    rc = fn(*([fake] * 17), None, None, fake, 1024, 2, 4, 64, 8, 1, *strides, 0, 0, 2, 0, 2, 0, None)
    assert rc < 0 and b"workspace" in lib.ak_last_error()
    rc = fn(*([fake] * 17), None, None, fake, 1 << 30, 2, 4, 64, 8, 1, *strides, 0, 0, 2, 3, 2, 0, None)
    assert rc == -2 and b"dtype" in lib.ak_last_error()  # delta neither fp32 nor u's type


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setenv("AUTOKERNEL_GFX950_LIB", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.HipExtensionMissing):
        _lib.load()


def test_row_extent_checks(lib):
    # The row kernels walk rows by grid stride on a capped grid, so the row
    # count is limited only by 64-bit addressing of the last row.
    huge = 1 << 61
    rc = lib.ak_rmsnorm_fwd(None, None, None, huge, 8, 8, 8, 1e-6, 0, None)
    assert rc == -1 and b"64-bit" in lib.ak_last_error()
    rc = lib.ak_fused_add_rmsnorm_fwd(None, None, None, None, None, 1 << 40, 8, 1 << 30, 8, 8, 8,
                                      1e-6, 1, None)
    assert rc == -1 and b"64-bit" in lib.ak_last_error()
    rc = lib.ak_softmax_fwd(None, None, huge, 8, 8, 8, 1, None)
    assert rc == -1 and b"64-bit" in lib.ak_last_error()
    rc = lib.ak_ce_fwd(None, None, None, None, None, None, None, huge, 8, 8, 8, 0.0, -100, 0.0,
                       1.0, 0.0, None, 2, None)
    assert rc == -1 and b"64-bit" in lib.ak_last_error()
    # 2^32 rows (past the old grid-size limit) pass the shape checks and stop
    # at the null-pointer check, before any HIP call
    for rows in (1 << 32, (1 << 32) + 5):
        rc = lib.ak_rmsnorm_fwd(None, None, None, rows, 8, 8, 8, 1e-6, 0, None)
        assert rc == -1 and b"null" in lib.ak_last_error()
        rc = lib.ak_softmax_fwd(None, None, rows, 8, 8, 8, 2, None)
        assert rc == -1 and b"null" in lib.ak_last_error()


def test_ce_reduction_argument_errors(lib):
    rc = lib.ak_ce_count_valid(None, 4, -100, None, None)
    assert rc == -1 and b"null" in lib.ak_last_error()
    rc = lib.ak_ce_mean(None, None, None, -1, -100, 0.0, None, None, None)
    assert rc == -1 and b"rows" in lib.ak_last_error()
    rc = lib.ak_ce_mean(None, None, None, 4, -100, -1.0, None, None, None)
    assert rc == -1 and b"z_loss" in lib.ak_last_error()
    rc = lib.ak_ce_bwd_tiny(None, None, None, None, None, 0, 8, 8, 8, 0.0, -100, 0.0, 1.0, -0.5,
                            None, 2, None)
    assert rc == -1 and b"z_loss" in lib.ak_last_error()


def test_no_alloc_entry_rejects_beyond_its_scratch(lib):
    # 256 partial rows x 16392 fp32 columns need more than the fixed 16 MiB;
    # the size check runs before the pointer checks and any HIP call
    rc = lib.ak_fused_add_rmsnorm_bwd_noalloc(None, None, None, None, None, ctypes.c_void_p(16),
                                              512, 16392, 16392, 16392, 16392, 16392, 1e-6, 0, None)
    assert rc == -4 and b"scratch" in lib.ak_last_error()
    # exactly 16 MiB (256 x 16384 fp32) passes the size check, then the null check
    rc = lib.ak_fused_add_rmsnorm_bwd_noalloc(None, None, None, None, None, ctypes.c_void_p(16),
                                              512, 16384, 16384, 16384, 16384, 16384, 1e-6, 0, None)
    assert rc == -1 and b"null" in lib.ak_last_error()


def _scan_fwd_args(dstate=16, bc_flags=0, bc_dtype=2, a_dtype=0, batch=0):
    # batch 0: every argument check runs, then the call returns before any HIP work
    return ([None] * 13 + [batch, 8, 64, dstate, 1] + [0] * 15
            + [1, bc_flags, 2, 0, bc_dtype, a_dtype, None])


def test_selective_scan_argument_contract(lib):
    f = lib.ak_selective_scan_fwd
    assert f(*_scan_fwd_args(dstate=256)) == 0            # the reference binding's limit
    assert f(*_scan_fwd_args(dstate=64, bc_flags=3)) == 0  # input-independent B and C
    rc = f(*_scan_fwd_args(dstate=257))
    assert rc == -2 and b"256" in lib.ak_last_error()
    assert f(*_scan_fwd_args(a_dtype=3)) == 0              # complex64 A
    rc = f(*_scan_fwd_args(a_dtype=1))
    assert rc == -2 and b"complex64" in lib.ak_last_error()
    rc = f(*_scan_fwd_args(a_dtype=3, batch=2))           # complex, real shape: null pointers
    assert rc == -1 and b"null" in lib.ak_last_error()
    rc = f(*_scan_fwd_args(bc_flags=4))                   # AK_SCAN_A_COMPLEX: workspace query only
    assert rc == -1 and b"bc_flags" in lib.ak_last_error()
    rc = f(*_scan_fwd_args(batch=2))                      # real shape: null pointers
    assert rc == -1 and b"null" in lib.ak_last_error()
    ws = lib.ak_selective_scan_bwd_workspace_bytes
    var, kb = ws(4, 2048, 4096, 64, 1, 0), ws(4, 2048, 4096, 64, 1, 1)
    # a constant B drops its [tiles, batch, groups, dstate, seqlen] partial rows
    # and keeps a [batch, dim, dstate] one instead
    tiles = 2048 // 16
    assert var - kb == tiles * 4 * 64 * 4096 * 4 - 4 * 2048 * 64 * 4
    # complex A: complex states every 16 steps, the pre-gate output (fp32 slots),
    # per-4-channel partial rows of (re, im) pairs, complex per-batch partials
    cw = ws(4, 2048, 4096, 64, 1, 4)
    a256 = lambda v: (v + 255) // 256 * 256
    assert cw == (a256(4 * 256 * 2048 * 64 * 8) + a256(4 * 2048 * 4096 * 4)
                  + 2 * a256(512 * 4 * 64 * 2 * 4096 * 4) + a256(4 * 2048 * 64 * 8) + 2 * a256(4 * 2048 * 4))
