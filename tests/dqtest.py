"""Shared test inputs and tolerances (not a test module).

Input recipes follow the reference's own tests:
  random block bytes with fp16 scales in U(0.002, 0.02)   test_int_kernels.cpp:44-61
  edge Q4_K blocks: d = 0 every 7th, saturated 6-bit scales every 11th
                                                            q4k_reference.h:69-87
  activations N(0,1) with outliers, an all-zero 32-block   test_qmm.cpp:78-89
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O

TYPES = (O.Q8_0, O.Q4_0, O.Q4_K, O.Q6_K)
BLOCK = {O.Q8_0: (32, 34), O.Q4_0: (32, 18), O.Q4_K: (256, 144), O.Q6_K: (256, 210)}
# (weight type, activation format) pairs with GPU kernels
PAIRS = [(O.Q8_0, O.ACT_PER32), (O.Q8_0, O.ACT_Q8_0), (O.Q4_0, O.ACT_PER32), (O.Q4_0, O.ACT_Q8_0),
         (O.Q4_K, O.ACT_Q8_K), (O.Q4_K, O.ACT_PER32), (O.Q6_K, O.ACT_Q8_K), (O.Q6_K, O.ACT_PER32)]

# fp32 parity bar: max relative error 1e-4, absolute 1e-5 near zero.
RTOL = 1e-4
ATOL = 1e-5


def pair_id(p) -> str:
    return f"{O.TYPE_NAMES[p[0]]}x{O.ACT_NAMES[p[1]]}"


def weight_rows(dtype: int, rows: int, k: int, seed: int, edge: bool = False) -> np.ndarray:
    """Random block bytes with valid small fp16 scales; `edge` adds the reference's
    edge blocks (d = 0, saturated scales, negative scales)."""
    w = O.random_bytes(seed, rows * O.row_bytes(dtype, k)).reshape(rows, -1).copy()
    rng = np.random.default_rng(seed)
    be, bb = BLOCK[dtype]
    nbk = k // be
    scales = O.fp32_to_fp16(rng.uniform(0.002, 0.02, (rows, nbk, 2)).astype(np.float32))
    if edge:
        sign = np.where(rng.integers(0, 2, scales.shape) == 1, np.uint16(0x8000), np.uint16(0))
        scales = scales | sign
    hb = scales.view(np.uint8).reshape(rows, nbk, 4)
    for b in range(nbk):
        o = b * bb
        if dtype == O.Q6_K:
            w[:, o + 208:o + 210] = hb[:, b, :2]
        elif dtype == O.Q4_K:
            w[:, o:o + 4] = hb[:, b, :]
        else:
            w[:, o:o + 2] = hb[:, b, :2]
    if edge:
        flat = w.reshape(rows * nbk, bb)
        for i in range(flat.shape[0]):
            if i % 7 == 3:  # d = 0
                if dtype == O.Q6_K:
                    flat[i, 208:210] = 0
                else:
                    flat[i, 0:2] = 0
            if i % 11 == 5 and dtype == O.Q4_K:  # saturated 6-bit scales and mins
                flat[i, 4:16] = 0xFF
            if i % 11 == 5 and dtype == O.Q6_K:  # extreme signed scales
                flat[i, 192:208] = np.array([0x80, 0x7F] * 8, np.uint8)
    return w


def activations(rows: int, k: int, seed: int, outliers: bool = True) -> np.ndarray:
    """N(0,1) rows; with outliers: 1% at 8 sigma, 3 channels at 40 sigma, and an
    all-zero 32-block in every third row (test_qmm.cpp:78-89)."""
    x = O.normal(seed, rows * k, outlier_frac=0.01 if outliers else 0.0, outlier_sigma=8.0).reshape(rows, k)
    if outliers:
        rng = np.random.default_rng(seed)
        for r in range(rows):
            for _ in range(3):
                x[r, rng.integers(0, k)] = np.float32(40.0 * rng.standard_normal())
            if k >= 64 and r % 3 == 1:
                x[r, 32:64] = 0.0
    return np.ascontiguousarray(x, dtype=np.float32)


def gguf_weights(dtype: int, n: int, k: int, seed: int, outlier_frac: float = 0.0) -> np.ndarray:
    """Weights N(0, 0.02) (optionally with outliers at 8 sigma) encoded as dtype."""
    w = O.normal(seed, n * k, std=0.02, outlier_frac=outlier_frac, outlier_sigma=8.0).reshape(n, k)
    return O.encode_weight(dtype, w)


def close(got: np.ndarray, want: np.ndarray, rtol: float = RTOL, atol: float = ATOL) -> tuple[bool, float]:
    """|got - want| <= max(rtol * |want|, atol) elementwise; returns (ok, worst ratio)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bound = np.maximum(rtol * np.abs(want), atol)
    ratio = np.abs(got - want) / bound
    worst = float(ratio.max()) if ratio.size else 0.0
    return bool(worst <= 1.0), worst
