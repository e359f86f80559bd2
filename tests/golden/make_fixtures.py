"""Generate the small numeric golden vectors of the fused linear contract.

The expected outputs come from the fp64 C brute force in oracle/gemm_ref.c
(an implementation independent of torch).  Cases cover the epilogue
variants and operand layouts of the kernel ABI on tiny, non-square shapes.
Run from the repo root: python tests/golden/make_fixtures.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle.fused_linear import brute_force  # noqa: E402

OUT = Path(__file__).resolve().parent / "fused_linear_small.npz"

CASES = [
    # (name, m, n, k, bias, activation, approximate)
    ("mm_1x17x9", 1, 17, 9, False, "none", "none"),
    ("addmm_31x65x33", 31, 65, 33, True, "none", "none"),
    ("gelu_erf_7x24x32", 7, 24, 32, True, "gelu", "none"),
    ("gelu_tanh_16x24x32", 16, 24, 32, True, "gelu", "tanh"),
    ("gelu_erf_nobias_33x40x19", 33, 40, 19, False, "gelu", "none"),
    ("relu_12x30x11", 12, 30, 11, True, "relu", "none"),
]


def main() -> None:
    rng = np.random.default_rng(20261201)
    arrays = {}
    for name, m, n, k, bias, act, approx in CASES:
        a = rng.standard_normal((m, k))
        w = rng.standard_normal((n, k))
        b = rng.uniform(-0.5, 0.5, n) if bias else None
        out = brute_force(a, w.T, b, act, approx)
        arrays[f"{name}/a"] = a
        arrays[f"{name}/w"] = w
        if b is not None:
            arrays[f"{name}/bias"] = b
        arrays[f"{name}/expected"] = out
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
