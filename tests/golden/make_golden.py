# SPDX-License-Identifier: Unlicense
"""Write tests/golden/ops_check_golden.npz: torch float64 outputs of the
reference's 33 generic-op cases (tests/ops_check.c:448-487 of
i.coregistration.opencl) on their exact inputs (the xorshift64 stream of
ops_check.c:33-42), by the closed forms of tests/ops_compare.py:73-235
(restated in tests/opcases.py, not imported).

The inputs are not stored: tests regenerate them bit-exactly from the
seed. The outputs are stored as float32 (the comparisons are at 2e-5
relative, far above float32 rounding).

    python tests/golden/make_golden.py
"""

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

import opcases  # noqa: E402


def main():
    out = {}
    for c in opcases.all_cases():
        for name, v in opcases.golden64(c).items():
            out[f"{c.name}/{name}"] = v.reshape(-1).numpy().astype(np.float32)
    np.savez_compressed(HERE / "ops_check_golden.npz", **out)
    print(f"{len(out)} outputs written to {HERE / 'ops_check_golden.npz'}")


if __name__ == "__main__":
    main()
