"""AutoKernel on MI355X (gfx950): swap model modules for gfx950 HIP kernels.

Usage (same surface as the reference ``autokernel/__init__.py``)::

    import autokernel
    model = autokernel.optimize(model)      # detect and apply every pattern
    print(autokernel.report(model))         # what was replaced
    autokernel.restore(model)               # put the original modules back
    autokernel.list_patterns()              # available pattern names
"""

from autokernel._registry import list_patterns, optimize, report, restore

__all__ = ["optimize", "report", "restore", "list_patterns"]
