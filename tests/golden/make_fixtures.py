"""Writes the known-answer fixtures used by tests/test_oracle.py.

The values are data held by the reference's own tests (no reference code is
run): the diagonal-scan known-answer test of
scripts/test_griffin_scan_op.py:42-52 (decay [.5, .8, .9, .7], value
[1, 2, 3, 4] -> [1.0, 2.8, 5.52, 7.864]) and the parameter grid of
external/mamba/tests/ops/test_selective_scan.py:15-51 with its tolerances
(:43-45).

Run: python tests/golden/make_fixtures.py
"""

import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))

FIXTURES = {
    "griffin_kat.json": {
        "source": "scripts/test_griffin_scan_op.py:42-52",
        "decay": [0.5, 0.8, 0.9, 0.7],
        "value": [1.0, 2.0, 3.0, 4.0],
        "expected": [1.0, 2.8, 5.52, 7.864],
    },
    "mamba_scan_grid.json": {
        "source": "external/mamba/tests/ops/test_selective_scan.py:15-51",
        "batch": 2,
        "dim": 4,
        "dstate": 8,
        "seqlen": [128, 256, 512, 1024, 2048, 4096],
        "varBC_groups": [1, 2],
        "has_D": True,
        "has_z": True,
        "has_delta_bias": True,
        "delta_softplus": True,
        "return_last_state": True,
        "tolerances": {"float32": [6e-4, 2e-3], "float16": [3e-3, 5e-3], "bfloat16": [3e-2, 5e-2]},
    },
}


def main():
    for name, payload in FIXTURES.items():
        with open(os.path.join(HERE, name), "w") as f:
            json.dump(payload, f, indent=1)
            f.write("\n")


if __name__ == "__main__":
    main()
