"""Writes tests/golden/select_matmul.npz: the reference's own select_matmul
(dynacore/src/kernel/matmul_registry.cpp:287-429, compiled from its sources into
oracle/_ref by `make -C oracle ref`) over a grid of shapes and KernelPlans, with the
MatmulCaps of a backend that has this library's kernels (oracle/ref_shim.cpp,
ref_select_matmul). Data only:

  plans    int32 [P, 9]: expand_min_rows, int8_decode_max_rows, int16_decode_max_rows,
           int8_superblock_min_rows, int8_superblock_max_rows, int8_subscale_min_rows,
           matmul_disabled (as int32 bits), qmm, qmm_gemm_min_rows
  cases    int64 [C, 6]: plan index, dtype, m, n, k, x_dense
  kernel   int32 [C]: MatmulKernelId
  act      int32 [C]: MatmulActFormat (kF32 0, kInt8Per32 1, kInt8Superblock 2,
           kInt8Subscaled 3, kInt16 4, kInt16Split 5)
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402

BIG = 1 << 30
DEFAULT = [2, 4, 0, 0, 8, 1, 0, 1, 9]  # KernelPlan::defaults(): qmm on, gemm from 9 rows
NOQMM = [2, 4, 0, 0, 8, 1, 0, 0, 9]    # the same without qmm (the x86 tiers' selection)
ENGINE = [2, BIG, 0, 0, 8, 1, 0, 1, 9]  # engine.cpp:365-375 on a qmm-accelerated backend


def ffn_down(p):
    """transformer.cpp:541-550 (int8_ffn_down off, int16_ffn_down on)."""
    d = list(p)
    if p[1] > 0:
        d[2] = max(p[1], p[4])
    d[1] = 0
    return d


PLANS = [
    DEFAULT,
    ffn_down(DEFAULT),
    NOQMM,
    ffn_down(NOQMM),
    ENGINE,
    ffn_down(ENGINE),
    [2, 4, 0, 1, 8, 1, 0, 0, 9],          # super-block opt-in (sub-scaled still first)
    [2, 4, 0, 1, 8, 0, 0, 0, 9],          # super-block instead of sub-scaled
    [2, BIG, 0, 1, BIG, 0, 0, 0, 9],      # every row on int8: the super-block class at any m
    [2, 64, 0, 0, 8, 1, 0, 0, 9],         # the NEON engine's int8 row limit
    ffn_down([2, 64, 0, 0, 8, 1, 0, 0, 9]),
    [2, 4, 0, 0, 8, 1, 1 << 7, 0, 9],     # sub-scaled disabled
    [2, 4, 0, 0, 8, 1, 1 << 9, 0, 9],     # per-32 disabled
    [2, 4, 8, 0, 8, 1, 1 << 13, 0, 9],    # int16 rows disabled
    [1, 4, 0, 0, 8, 1, 0, 0, 9],          # expand from one row
    [3, 0, 0, 0, 8, 1, 0, 0, 9],          # int8 decode off
    [2, 4, 16, 0, 8, 5, (1 << 7) | (1 << 8), 0, 9],
    [2, BIG, 0, 0, 8, 1, 1 << 1, 1, 9],   # qmm gemm disabled: qmm gemv at every size
    [2, BIG, 0, 0, 8, 1, 1 << 2, 1, 33],  # qmm gemv disabled, gemm from 33 rows
    [2, 4, 0, 0, 8, 1, (1 << 1) | (1 << 2), 1, 9],  # both qmm kernels disabled
    [2, 0, 16, 0, 8, 1, 0, 1, 4],         # int16 through qmm, gemm from 4 rows
]
TYPES = (6, 10, 14, 16)
MS = list(range(1, 21)) + [31, 32, 33, 63, 64, 65, 128, 512, 2048]


def main() -> None:
    r = O.ref()
    if r is None:
        raise SystemExit("build the reference first: make -C oracle ref")
    cases, kern, act = [], [], []
    for pi, p in enumerate(PLANS):
        for t in TYPES:
            for k in ((96, 4096, 14336) if t in (6, 10) else (256, 4096, 14336)):
                for m in MS:
                    for dense in (1, 0):
                        a = C.c_int(-1)
                        kid = r.ref_select_matmul(m, 4096, k, t, dense, *[int(v) for v in p[:6]],
                                                  C.c_uint32(p[6] & 0xFFFFFFFF), int(p[7]), int(p[8]), C.byref(a))
                        assert kid >= 0
                        cases.append((pi, t, m, 4096, k, dense))
                        kern.append(kid)
                        act.append(a.value)
    out = os.path.join(HERE, "select_matmul.npz")
    np.savez_compressed(out, plans=np.array(PLANS, np.int64).astype(np.int32), cases=np.array(cases, np.int64),
                        kernel=np.array(kern, np.int32), act=np.array(act, np.int32))
    print(out, len(cases), "cases", dict(zip(*np.unique(kern, return_counts=True))))


if __name__ == "__main__":
    main()
