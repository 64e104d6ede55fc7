"""GPU parity of the Q4_K x Q8_K GEMM on the f16 matrix cores (dq_gemm_h16.hip), on the
shapes the GEMM route sends to it: more than 128 activation rows and a grid of 128 x 256
tiles that reaches 5/8 of the CUs (N = 14336 and M > 256 on MI355X).

The kernel loads super-block s + 1's activation operands into a ring of two LDS buffers
while it runs super-block s, with one barrier per super-block. The cases cover what that
pipeline and the layout make distinct: super-block counts of 1 (no next load), 3 and 5,
a partial last activation tile, a row range that cuts the first and last weight tiles,
bias, both writers of the f16 operand layout (from Q8_K rows for dq_gemm, from fp32 rows
for dq_matmul), and saturated operands. Every output is bit-identical to the M=1 GEMV on
the same Q8_K rows and sampled columns to the oracle, except where saturated codes and
scales push a super-block's integer sum past 2^24: the fp32 accumulator then rounds, and
those outputs are held to a relative 2^-20 of the GEMV's (the GEMV sums in int32).

Reference style: dynacore/tests/test_qmm.cpp:178-282 (odd M, split ranges, tier equality).
"""
from __future__ import annotations

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import activations, weight_rows
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

N = 14336


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint32)


def _check(m: int, k: int, n0: int, n1: int, seed: int, saturate: bool = False) -> None:
    import dqtorch as T

    w_rows = weight_rows(O.Q4_K, N, k, seed, edge=True)
    if saturate:
        w_rows.reshape(N, k // 256, 144)[::5, :, 4:16] = 0xFF  # sc = m = 63
    a = O.quantize_act(O.ACT_Q8_K, activations(m, k, seed + 1))
    if saturate:
        a[0] = O.quantize_act(O.ACT_Q8_K, np.full((1, k), 3.0, np.float32))[0]
        a[m - 1] = O.quantize_act(O.ACT_Q8_K, np.full((1, k), -3.0, np.float32))[0]
    w = dq.Weight.upload(O.Q4_K, w_rows, k)
    bias = np.linspace(-2.5, 2.5, N, dtype=np.float32)
    ad, bd = dev(a), dev(bias)
    out = torch.full((m, N), 777.0, device="cuda")
    T.gemm(w, O.ACT_Q8_K, ad, n0=n0, n1=n1, bias=bd, out=out)
    yg = host(out)
    yv = host(T.gemv(w, O.ACT_Q8_K, ad, bias=bd))
    assert np.all(yg[:, :n0] == 777.0) and np.all(yg[:, n1:] == 777.0), "writes outside the row range"
    # rows whose super-block sums can pass 2^24 (the saturated +-3.0 rows): within a
    # relative 2^-20 of the GEMV; every other row bit-identical
    sat = [0, m - 1] if saturate else []
    exact = np.setdiff1d(np.arange(m), sat)
    assert np.array_equal(bits(yg[exact, n0:n1]), bits(yv[exact, n0:n1])), "GEMM differs from the GEMV"
    for r in sat:
        err = np.abs(yg[r, n0:n1].astype(np.float64) - yv[r, n0:n1])
        assert np.all(err <= 2.0**-20 * np.abs(yv[r, n0:n1]) + 1e-6), f"row {r}: max error {err.max()}"
    cols = np.random.default_rng(seed).choice(np.arange(n0, n1), 48, replace=False)
    want = O.matmul(O.Q4_K, O.ACT_Q8_K, w_rows[cols], a, k, bias[cols])
    assert np.array_equal(bits(yg[exact][:, cols]), bits(want[exact])), "GEMM differs from the oracle"
    if n0 == 0 and n1 == N:
        # dq_matmul: fp32 rows quantized straight into the f16 operand layout
        x = activations(m, k, seed + 1)
        ym = host(T.matmul(w, dev(x), bias=bd))
        yq = host(T.gemm(w, O.ACT_Q8_K, dev(O.quantize_act(O.ACT_Q8_K, x)), bias=bd))
        assert np.array_equal(bits(ym), bits(yq)), "dq_matmul differs from quantize + dq_gemm"


@pytest.mark.parametrize("m,k", [(300, 256), (384, 768), (520, 1280)])
def test_h16_superblock_counts(cuda, m, k):
    """1, 3 and 5 super-blocks (no next super-block to load; odd counts through the ring
    of two); m = 300 and 520 end on a partial activation tile (44 and 8 rows)."""
    _check(m, k, 0, N, 5100 + m)


def test_h16_row_range(cuda):
    """A row range that starts inside the first 64-row group and ends inside the last
    256-row weight tile: the kernel computes whole tiles and stores only [n0, n1)."""
    _check(400, 1024, 37, 14300, 5200)


def test_h16_saturated(cuda):
    """Saturated 6-bit scales and mins in every fifth weight row, activation rows of
    +127 and -127 codes: S and the mins term at their largest magnitudes (S past 2^24
    in the two saturated rows)."""
    _check(272, 512, 0, N, 5300, saturate=True)
