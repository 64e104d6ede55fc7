"""Writes tests/golden/qmm_vectors.npz: qmm activation buffers from the reference's own
ActBuffer::prepare / quantize_rows and its reference tier's quantize_row
(dynacore/cpu/qmm/qmm_reference.cpp:25-51,440-488), compiled into oracle/_ref by
`make -C oracle ref`. Inputs (rows with NaN, +-Inf, zero and tie values) and outputs only.

    python tests/golden/make_qmm_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as O  # noqa: E402


def rows(m: int, k: int, seed: int) -> np.ndarray:
    x = (np.random.default_rng(seed).standard_normal((m, k)) * 3).astype(np.float32)
    x[0, 3] = np.nan
    x[m - 1, 40] = np.inf
    x[m - 1, 0] = -np.inf
    x[0, 64:96] = 0.0
    x[0, 96:128] = -0.0
    x[m - 1, 32] = 127.0
    x[m - 1, 33:64] = np.float32(0.5) + np.arange(31, dtype=np.float32)
    return x


def main() -> None:
    out = {}
    x = rows(3, 256, 2024)
    out["x"] = x
    for mode in (0, 1):
        for paired in (0, 1):
            hi, lo, d, c = O.ref_qmm_quantize(x, mode, bool(paired))
            key = f"m{mode}p{paired}"
            out[f"{key}_hi"], out[f"{key}_d"], out[f"{key}_c"] = hi, d, c
            if lo is not None:
                out[f"{key}_lo"] = lo
    path = os.path.join(HERE, "qmm_vectors.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, sum(v.nbytes for v in out.values()), "bytes")


if __name__ == "__main__":
    main()
