"""AutoKernel -- drop-in for mamba_ssm's compiled ``selective_scan_cuda``
binding on gfx950.

``fwd`` and ``bwd`` keep the argument order and return lists of the
reference binding (``external/mamba/csrc/selective_scan/selective_scan.cpp:
227-335`` and ``:339-490``, registered at ``:492-497``), so code written
against it -- ``SelectiveScanFn`` and ``mamba_inner_fn`` in
``external/mamba/mamba_ssm/ops/selective_scan_interface.py`` -- can import
this module in its place::

    from kernels.hip import selective_scan_cuda

The binding's contract is kept: ``dstate <= 256``
(``selective_scan.cpp:262``), input-dependent ``B`` / ``C`` (``[batch,
dstate, seqlen]`` or ``[batch, ngroups, dstate, seqlen]``) or
input-independent ones (``[dim, dstate]`` fp32, ``:115-121``), and the
gradients of input-dependent ``B`` / ``C`` summed in fp32 and returned in
their dtype (``:461``, ``:488``; an input-independent one is fp32). Complex
weights (``A`` complex64, ``:236-240``) take input-dependent ``B`` / ``C`` as
real ``[batch, (ngroups,) dstate, 2 * seqlen]`` (``:270-276``) or
input-independent complex ones; ``x``, ``dA`` and a constant ``dB`` / ``dC``
are then complex64.

Differences, by design: the backward recomputes the states itself, so the
chunk-state tensor ``x`` and the forward output ``out`` passed to ``bwd`` are
accepted and not read; ``delta`` may be fp32 with half-precision ``u``.
"""

from kernels.hip.selective_scan import _normalise, _scan_backward, _scan_forward


def fwd(u, delta, A, B, C, D_=None, z_=None, delta_bias_=None, delta_softplus=False):
    """``[out, x]``, or ``[out, x, out_z]`` with a gate ``z``.

    ``out``: y + D u in u's dtype (before the gate); ``x``: fp32 (complex64
    with a complex ``A``) ``[batch, dim, n_chunks, 2 * dstate]``, per
    2048-step chunk the running prefix (prod exp(delta' A), state) of each
    state, interleaved;
    ``out_z``: ``out * silu(z)``.
    """
    gated = z_ is not None
    out, _, _, prez, chunks = _scan_forward(u, delta, A, B, C, D_, z_, delta_bias_, delta_softplus,
                                            False, want_prez=gated, want_chunk_states=True)
    x = chunks.view(chunks.shape[0], chunks.shape[1], chunks.shape[2], -1)
    if gated:
        return [prez, x, out]
    return [out, x]


def bwd(u, delta, A, B, C, D_, z_, delta_bias_, dout, x_, out_, dz_, delta_softplus,
        recompute_out_z):
    """``[du, ddelta, dA, dB, dC, dD, ddelta_bias]``, then ``dz`` with a gate,
    then ``out_z`` when ``recompute_out_z``. ``dD`` / ``ddelta_bias`` are None
    without ``D`` / ``delta_bias``; ``dz_`` (optional) receives dz in place."""
    del x_, out_
    args = _normalise(u, delta, A, B, C, D_, z_, delta_bias_)
    du, ddelta, dA, dB, dC, dD, dz, dbias = _scan_backward(dout, *args, delta_softplus)
    if B.dim() == 3:
        dB = dB.squeeze(1)
    if C.dim() == 3:
        dC = dC.squeeze(1)
    res = [du, ddelta.to(delta.dtype), dA.to(A.dtype), dB.to(B.dtype), dC.to(C.dtype),
           dD.to(D_.dtype) if dD is not None else None,
           dbias.to(delta_bias_.dtype) if dbias is not None else None]
    if z_ is not None:
        if dz_ is not None:
            dz_.copy_(dz)
            dz = dz_
        res.append(dz)
    if recompute_out_z:
        out_z, _, _ = _scan_forward(u, delta, A, B, C, D_, z_, delta_bias_, delta_softplus, False)
        res.append(out_z)
    return res
