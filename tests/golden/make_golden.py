"""Writes tests/golden/reference_vectors.npz from the reference's own CPU kernels.

Run in a container where /root/reference exists and `make -C oracle ref` has
built oracle/_ref/libdynacore_ref.so (the reference's sources compiled as they
lie; see oracle/Makefile). The fixture holds inputs and the reference's outputs
only (data, no code):

  fp16         fp16 -> fp32 of all 65,536 half values; fp32 -> fp16 of boundary values
  act_*        quantized activation bytes of seeded rows:
               q8_0 (quantize_q8_0, quant_formats.cpp:60-74), per32 (generic
               quantize_act, kernels_generic.cpp:187-207), sb (quantize_act_sb,
               kernels_avx2.cpp:638-644), sx (quantize_act_sx, kernels_avx2.cpp:1077-1096)
  deq_<t>      dequantize_<t> of random block bytes (quant_formats.cpp:12-222)
  dot_<t>      generic dot_rows_<t> (kernels_generic.cpp:216-310) on per-32 activations
  sbdot_<t>    AVX2 dot_rows_sb_<t> (kernels_avx2.cpp:976-1058), sxdot_<t> AVX2
               dot_rows_sx_<t> (kernels_avx2.cpp:1117-1216)
  expnp        exp_nonpos of seeded and boundary inputs (base/fast_exp.h:16-35), the
               exponential of the reference's SiLU (cpu_device.cpp:117-123)
  q16_x, act_q16  int16 activations (AVX2 quantize_act16, kernels_avx2.cpp:1631-1652) of
               the act_x rows and of an edge row (ties, a zero block, +-inf, full-scale
               codes); split_q16 their split_act16 bytes (kernels_generic.cpp:334-346)
  q16dot_<t>   AVX2 dot_rows16_<t> (kernels_avx2.cpp:1662-1765) on act_q16, t in
               q8_0, q4_K, q6_K
  vecdot_<t>   generic vec_dot_<t> (kernels_generic.cpp:67-150) of the w_<t> rows and the
               fp32 act_x rows (the kF32 contract, no activation quantization)
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402

K = 512
ROWS = 4
TYPES = (O.Q8_0, O.Q4_0, O.Q4_K, O.Q6_K)


def weight_rows(dtype: int, rows: int, k: int, seed: int) -> np.ndarray:
    """Random block bytes with fp16 scales in U(0.002, 0.02) (test_int_kernels.cpp:44-61)."""
    w = O.random_bytes(seed, rows * O.row_bytes(dtype, k)).reshape(rows, -1).copy()
    rng = np.random.default_rng(seed)
    be = 32 if dtype in (O.Q8_0, O.Q4_0) else 256
    bb = {O.Q8_0: 34, O.Q4_0: 18, O.Q4_K: 144, O.Q6_K: 210}[dtype]
    for r in range(rows):
        for b in range(k // be):
            o = b * bb
            h = O.fp32_to_fp16(rng.uniform(0.002, 0.02, 2).astype(np.float32)).view(np.uint8)
            if dtype == O.Q6_K:
                w[r, o + 208:o + 210] = h[:2]
            elif dtype == O.Q4_K:
                w[r, o:o + 4] = h
            else:
                w[r, o:o + 2] = h[:2]
    return w


def activations(rows: int, k: int, seed: int) -> np.ndarray:
    """N(0,1) with 1% outliers at 8 sigma, an all-zero 32-block and exact-tie values."""
    x = O.normal(seed, rows * k, outlier_frac=0.01, outlier_sigma=8.0).reshape(rows, k)
    x[1, 32:64] = 0.0
    # x * (127 / amax) lands exactly on k + 0.5 for these: amax = 127 -> id = 1
    x[2, 64:96] = np.linspace(-15.5, 15.5, 32, dtype=np.float32)
    x[2, 64] = 127.0
    return np.ascontiguousarray(x, dtype=np.float32)


def q16_edge_row(k: int) -> np.ndarray:
    """Edge cases of the int16 quantizer: x * (32767 / amax) on exact ties (amax =
    32767 gives id = 1), a zero block, a block with +inf and -inf (d = inf, id = 0),
    full-scale values of both signs, tiny values."""
    x = O.normal(77, k).astype(np.float32)
    x[0:32] = np.concatenate([np.arange(-7.5, 8.5, 1.0), np.arange(100.5, 116.5, 1.0)]).astype(np.float32)
    x[0] = -32767.0
    x[32:64] = 0.0
    x[64 + 5] = np.inf
    x[64 + 9] = -np.inf
    x[96:128] = np.where(np.arange(32) % 2 == 0, 1.0, -1.0).astype(np.float32) * np.float32(3.0e4)
    x[128:160] *= np.float32(1e-30)
    return x


def main() -> None:
    r = O.ref()
    if r is None:
        raise SystemExit("oracle/_ref is not built (make -C oracle ref)")
    out: dict[str, np.ndarray] = {}
    h = np.arange(65536, dtype=np.uint16)
    out["fp16_h"] = h
    out["fp16_f"] = np.array([r.ref_fp16_to_fp32(int(v)) for v in h], np.float32)
    f = np.concatenate([
        out["fp16_f"][np.isfinite(out["fp16_f"])],
        (out["fp16_f"][np.isfinite(out["fp16_f"])].astype(np.float64) * (1 + 2.0 ** -11)).astype(np.float32),
        np.array([65504, 65519.99, 65520, 65536, 1e-8, 2.0 ** -25, 2.0 ** -24 * 1.5, -0.0, np.inf, -np.inf, np.nan],
                 np.float32),
    ])
    out["f2h_f"] = f
    out["f2h_h"] = np.array([r.ref_fp32_to_fp16(float(v)) for v in f], np.uint16)

    x = activations(ROWS, K, 20261201)
    out["act_x"] = x
    for kind in ("q8_0", "per32", "sb", "sx"):
        out[f"act_{kind}"] = np.stack([O.ref_quantize(kind, x[i]) for i in range(ROWS)])

    for t in TYPES:
        name = O.TYPE_NAMES[t]
        w = weight_rows(t, 3, K, 1000 + t)
        out[f"w_{name}"] = w
        out[f"deq_{name}"] = np.stack([O.ref_dequantize(t, w[i], K) for i in range(3)])
        per32 = out["act_per32"]
        out[f"dot_{name}"] = np.stack([O.ref_dot_rows(0, t, w[i], per32, K) for i in range(3)], 1)
        if t in (O.Q4_K, O.Q6_K):
            out[f"sbdot_{name}"] = np.stack([O.ref_dot_rows(2, t, w[i], out["act_sb"], K) for i in range(3)], 1)
            out[f"sxdot_{name}"] = np.stack([O.ref_dot_rows(3, t, w[i], out["act_sx"], K) for i in range(3)], 1)

    q16x = np.concatenate([x, q16_edge_row(K)[None]], 0)
    out["q16_x"] = q16x
    out["act_q16"] = np.stack([O.ref_quantize("q16", row) for row in q16x])
    out["split_q16"] = np.stack([O.ref_split_act16(a) for a in out["act_q16"]])
    for t in (O.Q8_0, O.Q4_K, O.Q6_K):
        name = O.TYPE_NAMES[t]
        w = out[f"w_{name}"]
        dots = [O.ref_dot_rows16(t, w[i], out["act_q16"][r0:r0 + 4], K) for i in range(3) for r0 in (0, 4)]
        out[f"q16dot_{name}"] = np.stack([np.concatenate(dots[2 * i:2 * i + 2]) for i in range(3)], 1)

    for t in TYPES:
        name = O.TYPE_NAMES[t]
        out[f"vecdot_{name}"] = np.array([[O.ref_vec_dot(0, t, out[f"w_{name}"][i], x[r], K) for i in range(3)]
                                          for r in range(ROWS)], np.float32)

    rng = np.random.default_rng(20261202)
    ex = np.concatenate([
        -rng.exponential(6.0, 4096), -rng.uniform(0.0, 1.0, 1024), np.linspace(-90.0, 0.0, 1801),
        np.array([0.0, -0.0, -87.0, -86.99999, -87.00001, -88.0, -100.0, -1e-30, -1e-45, -np.log(2.0), 1.0, 88.0,
                  100.0, -np.inf, np.nan]),
    ]).astype(np.float32)
    out["expnp_x"] = ex
    out["expnp_y"] = np.array([r.ref_exp_nonpos(float(v)) for v in ex], np.float32)
    path = os.path.join(HERE, "reference_vectors.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
