"""GPU parity of the Q4_K x int16 GEMM on the f16 matrix cores (dq_gemm_q16.hip): the
int16 contract (ActBlockQ16 rows: int16 codes, one scale and one code sum per 32
values; dynacore/cpu/avx2/kernels_avx2.cpp:1631-1729) through dq_gemm on DQ_ACT_Q16
rows, dq_matmul_act(DQ_ACT_Q16) on fp32 rows and dq_qmm_gemm in int16 mode, which
take it from 5 rows (split K where its tiles leave CUs idle).

The integers sc_j P_j are rounded to fp32 where they pass 2^24 and the fp32 terms are
summed in an order of the kernel's own, so it is held to the reference's bound against
the exact product, |y - y_exact| <= 1e-5 * sum |w_i x_i|
(dynacore/tests/test_int_kernels.cpp:131-147), and to the int16 GEMV's bar against the
oracle's int16 order (and, for qmm, the reference build's qmm gemv), |y - y_oracle| <=
2e-6 * sum |w_i x_i|. A bar relative to the output does not fit this contract: its
order keeps the products and the mins term as two sums that cancel, each carrying
~1e-5 of fp32 rounding at K = 4096 for outputs of order 1, so two correct orders
differ by more than 1e-5 absolute near zero.

Cases: 1, 5 and 16 super-blocks, partial and whole 32- and 64-row activation tiles
(dq_matmul_act's first GEMM row count included), a row range cutting
the first and last 256-row weight tiles, bias, saturated scales and codes of +-32767,
the reference's edge blocks, and both writers' routes (dq_gemm on int16 rows,
dq_matmul_act on fp32 rows), which must agree bit for bit.

Reference style: dynacore/tests/test_qmm.cpp:178-282 (odd M, split ranges, tier equality).
"""
from __future__ import annotations

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import activations, gguf_weights, weight_rows
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint32)


def _bound(w_rows: np.ndarray, a: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    wf = O.dequantize(O.Q4_K, w_rows, k).astype(np.float64)
    af = O.dequantize_act(O.ACT_Q16, a, k).astype(np.float64)
    return af @ wf.T, np.abs(af) @ np.abs(wf).T


def _check(m: int, k: int, n: int, n0: int, n1: int, seed: int, saturate: bool = False, stress: bool = False) -> None:
    import dqtorch as T

    if stress:
        w_rows = weight_rows(O.Q4_K, n, k, seed, edge=True)
    else:
        w_rows = gguf_weights(O.Q4_K, n, k, seed, outlier_frac=0.01)
    if saturate:
        w_rows.reshape(n, k // 256, 144)[::5, :, 4:16] = 0xFF  # sc = m = 63
    x = activations(m, k, seed + 1, outliers=stress)
    if saturate:
        x[0] = 3.0  # every code 32767
        x[m - 1] = -3.0
    a = O.quantize_act(O.ACT_Q16, x)
    w = dq.Weight.upload(O.Q4_K, w_rows, k)
    bias = np.linspace(-2.5, 2.5, n, dtype=np.float32)
    ad, bd = dev(a), dev(bias)
    out = torch.full((m, n), 777.0, device="cuda")
    T.gemm(w, O.ACT_Q16, ad, n0=n0, n1=n1, bias=bd, out=out)
    yg = host(out)
    assert np.all(yg[:, :n0] == 777.0) and np.all(yg[:, n1:] == 777.0), "writes outside the row range"
    exact, mag = _bound(w_rows, a, k)
    exact += bias
    err = np.abs(yg[:, n0:n1] - exact[:, n0:n1])
    assert np.all(err <= 1e-5 * mag[:, n0:n1] + 1e-6), f"worst {np.max(err / (1e-5 * mag[:, n0:n1] + 1e-6)):.3g}"
    want = O.matmul(O.Q4_K, O.ACT_Q16, w_rows, a, k, bias).astype(np.float64)
    d = np.abs(yg[:, n0:n1] - want[:, n0:n1])
    assert np.all(d <= 2e-6 * mag[:, n0:n1] + 1e-30), f"oracle: worst {np.max(d / (2e-6 * mag[:, n0:n1] + 1e-30)):.3g}"
    if n0 == 0 and n1 == n:
        # fp32 rows: quantized to int16 rows and converted inside dq_matmul_act
        ym = host(T.matmul_act(w, O.ACT_Q16, dev(x), bias=bd))
        assert np.array_equal(bits(ym), bits(yg)), "dq_matmul_act differs from dq_gemm on the same rows"
    w.free()


@pytest.mark.parametrize("m,k", [(24, 256), (67, 1280), (130, 4096)])
def test_q16_gemm_superblock_counts(cuda, m, k):
    """1, 5 and 16 super-blocks; 24, 67 and 130 rows end on partial activation tiles
    (32 rows per workgroup up to 32 rows, else 64)."""
    _check(m, k, 1024, 0, 1024, 9100 + m)


@pytest.mark.parametrize("m", [5, 32, 33])
def test_q16_gemm_tile_rows(cuda, m):
    """Around the switch from one 32-row activation tile per workgroup (m <= 32) to two:
    dq_matmul_act's first GEMM row count, a whole single tile, a second tile with one
    row; 8 weight tiles, each in 8 super-block ranges."""
    _check(m, 4096, 2048, 0, 2048, 9150 + m)


def test_q16_gemm_row_range(cuda):
    """A row range that starts inside the first 64-row group and ends inside the last
    256-row weight tile: whole tiles computed, only [n0, n1) stored."""
    _check(80, 1024, 1536, 37, 1500, 9200)


def test_q16_gemm_stress_and_saturated(cuda):
    """The reference's edge blocks (d = 0, saturated and negative scales, random bytes),
    saturated 6-bit scales and mins in every fifth row, and rows of +-32767 codes."""
    _check(72, 512, 1024, 0, 1024, 9300, saturate=True, stress=True)


def test_q16_gemm_bench_shape(cuda):
    """Config 4's shape (K=4096, N=14336) at M=512: 256 sampled columns against the
    exact product and the oracle."""
    import dqtorch as T

    m, k, n = 512, 4096, 14336
    w_rows = gguf_weights(O.Q4_K, n, k, 9400, outlier_frac=0.01)
    x = activations(m, k, 9401, outliers=False)
    w = dq.Weight.upload(O.Q4_K, w_rows, k)
    ym = host(T.matmul_act(w, O.ACT_Q16, dev(x)))
    a = O.quantize_act(O.ACT_Q16, x)
    cols = np.random.default_rng(9402).choice(n, 256, replace=False)
    exact, mag = _bound(w_rows[cols], a, k)
    assert np.all(np.abs(ym[:, cols] - exact) <= 1e-5 * mag)
    want = O.matmul(O.Q4_K, O.ACT_Q16, w_rows[cols], a, k).astype(np.float64)
    assert np.all(np.abs(ym[:, cols] - want) <= 2e-6 * mag)
    w.free()


@pytest.mark.parametrize("paired", [False, True])
def test_q16_qmm_gemm(cuda, paired):
    """dq_qmm_gemm in int16 mode on a qmm buffer of 150 rows: the GEMM on the buffer's
    blocks, within tolerance of the reference build's qmm gemv (its own fp32 order)."""
    m, k, n = 150, 1024, 512
    w_rows = gguf_weights(O.Q4_K, n, k, 9500, outlier_frac=0.01)
    x = activations(m, k, 9501, outliers=False)
    w = dq.Weight.upload(O.Q4_K, w_rows, k)
    nbytes = dq.qmm_act_bytes(dq.QMM_INT16, m, k, paired)
    buf = torch.empty((nbytes,), dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    acts = dq.qmm_act_prepare(buf, nbytes, dq.QMM_INT16, m, k, paired, st)
    dq.qmm_quantize_rows(dev(x), k, 0, m, acts, st)
    y = torch.zeros((m, n), device="cuda")
    dq.qmm_gemm(w, 0, n, acts, y, n, None, st)
    got = host(y)
    a = O.quantize_act(O.ACT_Q16, x)
    exact, mag = _bound(w_rows, a, k)
    assert np.all(np.abs(got - exact) <= 1e-5 * mag + 1e-6)
    if O.ref_available():
        ref = O.ref_qmm_gemv(O.Q4_K, w_rows, x, dq.QMM_INT16, paired).astype(np.float64)
        assert np.all(np.abs(got - ref) <= 2e-6 * mag + 1e-30)
    w.free()
