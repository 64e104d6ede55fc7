"""Writes tests/golden/expand_vectors.npz: the reference's fp32 expand + GEMM class
(dynacore's kF32ExpandGemm, cpu_device.cpp:1114-1152) on fixed inputs.

Run where /root/reference exists and `make -C oracle ref` has built
oracle/_ref/libdynacore_ref.so. Inputs are the golden rows of reference_vectors.npz
(w_<t> at K = 512, act_x) and seeded rows below; outputs come from the reference's
own x86 kernels (data only):

  exp_<t>          AVX2 dequant_<t> (kernels_avx2.cpp:370-466) of the w_<t> rows
  rw_<t>, exp_rw_<t>  24 seeded weight rows at K = 1056 (33 blocks of 32 for Q8_0 /
                   Q4_0, so a 64-value slice holds half a slice of zeros; K-quants at
                   1024) and the AVX2 expansion of the first 8
  expgemm_<t>      expand + gemm_panel (kernels_avx2.cpp:146-230) of act_x x w_<t>
  gx_<t>, expgemm_rw_<t>  20 seeded activation rows x the rw_<t> rows, same path
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402

TYPES = (O.Q8_0, O.Q4_0, O.Q4_K, O.Q6_K)


def main() -> None:
    if not O.ref_available() or not O.ref().ref_has_avx2():
        sys.exit("needs oracle/_ref built from /root/reference on an AVX2 host")
    g = np.load(os.path.join(HERE, "reference_vectors.npz"))
    out = {}
    for t in TYPES:
        name = O.TYPE_NAMES[t]
        w = g[f"w_{name}"]
        out[f"exp_{name}"] = O.ref_expand_x86(t, w, 512)
        out[f"expgemm_{name}"] = O.ref_expand_gemm(t, w, g["act_x"])
        k = 1024 if t in (O.Q4_K, O.Q6_K) else 1056
        rng = np.random.default_rng(4400 + t)
        vals = rng.normal(0.0, 0.02, (24, k)).astype(np.float32)
        vals[3] *= 40.0  # one row with large scales
        rw = O.encode_weight(t, vals)
        out[f"rw_{name}"] = rw
        out[f"exp_rw_{name}"] = O.ref_expand_x86(t, rw[:8], k)
        gx = np.random.default_rng(4500 + t).normal(0.0, 1.0, (20, k)).astype(np.float32)
        out[f"gx_{name}"] = gx
        out[f"expgemm_rw_{name}"] = O.ref_expand_gemm(t, rw, gx)
    np.savez_compressed(os.path.join(HERE, "expand_vectors.npz"), **out)
    print("wrote", os.path.join(HERE, "expand_vectors.npz"), sum(v.nbytes for v in out.values()), "bytes")


if __name__ == "__main__":
    main()
