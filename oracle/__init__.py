"""CPU oracle for the gfx950 kernels -- test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package. ``ops`` holds torch-CPU restatements of the
reference functions; ``c_oracle`` wraps the C restatement of the Mamba-1
scan (``scan_ref.c``, built by ``make -C oracle``).
"""
