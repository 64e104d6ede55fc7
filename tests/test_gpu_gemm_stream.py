"""GPU parity of the streamed Q4_K x Q8_K GEMM (dq_gemm_stream.hip), on the shapes the
GEMM route sends to it: more than 128 activation rows and a grid of 128 x 256 tiles
that reaches 5/8 of the CUs (N = 14336 and M > 256 on MI355X).

The kernel runs K in half super-blocks with the two waves of a SIMD half a super-block
apart, DMA loads two positions ahead into a ring of four buffers and per-super-block
data into a ring of three. The cases cover what that pipeline makes distinct: an odd
super-block count (the lagging waves finish on a first half), counts below and above
the ring depths (1, 3, 5 super-blocks), a partial last activation tile, a row range
that cuts the first and last weight tiles, bias, and saturated operands. Every output
is bit-identical to the M=1 GEMV on the same Q8_K rows, sampled columns to the oracle.

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
    assert np.array_equal(bits(yg[:, n0:n1]), bits(yv[:, n0:n1])), "GEMM differs from the GEMV"
    cols = np.random.default_rng(seed).choice(np.arange(n0, n1), 48, replace=False)
    want = O.matmul(O.Q4_K, O.ACT_Q8_K, w_rows[cols], a, k, bias[cols])
    assert np.array_equal(bits(yg[:, cols]), bits(want)), "GEMM differs from the oracle"


@pytest.mark.parametrize("m,k", [(300, 256), (384, 768), (520, 1280)])
def test_stream_superblock_counts(cuda, m, k):
    """1, 3 and 5 super-blocks (below the per-super-block ring depth, odd, above it);
    m = 300 and 520 end on a partial activation tile (44 and 8 rows)."""
    _check(m, k, 0, N, 5100 + m)


def test_stream_row_range(cuda):
    """A row range that starts inside the first 64-row group and ends inside the last
    256-row weight tile: the kernel computes whole tiles and stores only [n0, n1)."""
    _check(400, 1024, 37, 14300, 5200)


def test_stream_saturated(cuda):
    """Saturated 6-bit scales and mins in every fifth weight row, activation rows of
    +127 and -127 codes: S and the mins term at their largest magnitudes."""
    _check(272, 512, 0, N, 5300, saturate=True)
