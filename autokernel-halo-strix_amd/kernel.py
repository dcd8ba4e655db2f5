"""AutoKernel -- cross-entropy kernel facade (``import kernel``).

Re-exports the public API of ``kernels.ce_fused`` at the package root, as the
reference's ``kernel.py`` (:9-27) does for its bench harness and scripts.
"""
from kernels.ce_fused import *  # noqa: F401,F403
from kernels.ce_fused import (  # noqa: F401
    KERNEL_TYPE,
    BACKEND,
    MODEL_SHAPES,
    TEST_SIZES,
    TOLERANCES,
    FLOPS_FN,
    BYTES_FN,
    kernel_fn,
    ce_full,
    _get_fwd_module,
    _get_bwd_module,
    _CrossEntropyHIP,
    HIP_FWD_SRC,
    HIP_BWD_SRC,
)
