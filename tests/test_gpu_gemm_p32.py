"""GPU parity of the Q4_K x per-32 GEMM on the f16 matrix cores (dq_gemm_p32.hip), qmm's
int8 gemm contract: dq_gemm on DQ_ACT_PER32 rows, dq_matmul_act(DQ_ACT_PER32) and
dq_qmm_gemm in int8 mode send Q4_K from 5 rows to it (split K where its tiles leave
CUs idle).

Its per-sub-block integers P_j are exact; the fp32 terms are summed in an order of
its own (two VALU operations per output and sub-block, the mins term on fp32 MFMAs),
so it is held to the reference's bound against the exact product,
|y - y_exact| <= 1e-5 * sum |w_i x_i| (dynacore/tests/test_int_kernels.cpp:131-147), and
to the north-star tolerance (1e-4 relative, 1e-5 absolute) against the oracle's per-32
order and the reference build's qmm gemv. The cases cover super-block counts of 1, 3
and 5 through the ring of two LDS buffers, a partial last activation tile, a row range
that cuts the first and last weight tiles, bias, saturated scales and codes, and both
writers' routes (per-32 rows through dq_gemm, fp32 rows through dq_matmul_act), which
must agree bit for bit.

Reference style: dynacore/tests/test_qmm.cpp:178-282 (odd M, split ranges, tier equality).
"""
from __future__ import annotations

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import activations, close, gguf_weights, weight_rows
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
    af = O.dequantize_act(O.ACT_PER32, a, k).astype(np.float64)
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
        x[0] = 3.0
        x[m - 1] = -3.0
    a = O.quantize_act(O.ACT_PER32, x)
    w = dq.Weight.upload(O.Q4_K, w_rows, k)
    bias = np.linspace(-2.5, 2.5, n, dtype=np.float32)
    ad, bd = dev(a), dev(bias)
    out = torch.full((m, n), 777.0, device="cuda")
    T.gemm(w, O.ACT_PER32, ad, n0=n0, n1=n1, bias=bd, out=out)
    yg = host(out)
    assert np.all(yg[:, :n0] == 777.0) and np.all(yg[:, n1:] == 777.0), "writes outside the row range"
    exact, mag = _bound(w_rows, a, k)
    exact += bias
    err = np.abs(yg[:, n0:n1] - exact[:, n0:n1])
    assert np.all(err <= 1e-5 * mag[:, n0:n1] + 1e-6), f"worst {np.max(err / (1e-5 * mag[:, n0:n1] + 1e-6)):.3g}"
    if not stress:
        want = O.matmul(O.Q4_K, O.ACT_PER32, w_rows, a, k, bias)
        ok, worst = close(yg[:, n0:n1], want[:, n0:n1])
        assert ok, f"oracle: worst error ratio {worst:.3g}"
    if n0 == 0 and n1 == n:
        # fp32 rows: quantized to per-32 rows and converted inside dq_matmul_act
        ym = host(T.matmul_act(w, O.ACT_PER32, dev(x), bias=bd))
        assert np.array_equal(bits(ym), bits(yg)), "dq_matmul_act differs from dq_gemm on the same rows"
    w.free()


@pytest.mark.parametrize("m,k", [(300, 256), (130, 768), (520, 1280)])
def test_p32_superblock_counts(cuda, m, k):
    """1, 3 and 5 super-blocks; m = 300, 130 and 520 end on partial activation tiles."""
    _check(m, k, 2048, 0, 2048, 6100 + m)


def test_p32_split_ranges(cuda):
    """20 rows on 8 weight tiles (K = 4096): each tile's 16 super-blocks split into 8
    ranges whose partials a second launch adds in order; dq_gemm on the per-32 rows."""
    _check(20, 4096, 2048, 0, 2048, 6150)


@pytest.mark.parametrize("m", [5, 32, 33, 64, 65])
def test_p32_tile_rows(cuda, m):
    """Around the switches from one 32-row activation tile per workgroup (m <= 32) to two
    (m <= 64) and four: dq_matmul_act's first GEMM row count, whole tiles and one row past
    them; 8 weight tiles, each in 8 super-block ranges."""
    _check(m, 4096, 2048, 0, 2048, 6160 + m)


def test_p32_row_range(cuda):
    """A row range that starts inside the first 64-row group and ends inside the last
    256-row weight tile: the kernel computes whole tiles and stores only [n0, n1)."""
    _check(200, 1024, 1536, 37, 1500, 6200)


def test_p32_stress_and_saturated(cuda):
    """The reference's edge blocks (d = 0, saturated and negative scales, random bytes),
    saturated 6-bit scales and mins in every fifth row, and rows of +-127 codes."""
    _check(272, 512, 1024, 0, 1024, 6300, saturate=True, stress=True)


def test_p32_bench_shape(cuda):
    """Config 4 (K=4096, N=14336) at M=512: one round of 224 workgroups over 16
    super-blocks; 256 sampled columns against the exact product and the oracle."""
    import dqtorch as T

    m, k, n = 512, 4096, 14336
    w_rows = gguf_weights(O.Q4_K, n, k, 6400, outlier_frac=0.01)
    x = activations(m, k, 6401, outliers=False)
    w = dq.Weight.upload(O.Q4_K, w_rows, k)
    ym = host(T.matmul_act(w, O.ACT_PER32, dev(x)))
    a = O.quantize_act(O.ACT_PER32, x)
    cols = np.random.default_rng(6402).choice(n, 256, replace=False)
    exact, mag = _bound(w_rows[cols], a, k)
    assert np.all(np.abs(ym[:, cols] - exact) <= 1e-5 * mag)
    ok, worst = close(ym[:, cols], O.matmul(O.Q4_K, O.ACT_PER32, w_rows[cols], a, k))
    assert ok, f"worst error ratio {worst:.3g}"
    w.free()


@pytest.mark.parametrize("paired", [False, True])
def test_p32_qmm_gemm(cuda, paired):
    """dq_qmm_gemm in int8 mode on a qmm buffer of 150 rows: the GEMM on the buffer's
    blocks, within tolerance of the reference build's qmm gemv (its own fp32 order)."""
    m, k, n = 150, 1024, 512
    w_rows = gguf_weights(O.Q4_K, n, k, 6500, outlier_frac=0.01)
    x = activations(m, k, 6501, outliers=False)
    w = dq.Weight.upload(O.Q4_K, w_rows, k)
    nbytes = dq.qmm_act_bytes(dq.QMM_INT8, m, k, paired)
    buf = torch.empty((nbytes,), dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    acts = dq.qmm_act_prepare(buf, nbytes, dq.QMM_INT8, m, k, paired, st)
    xd = dev(x)
    dq.qmm_quantize_rows(xd, k, 0, m, acts, st)
    y = torch.zeros((m, n), device="cuda")
    dq.qmm_gemm(w, 0, n, acts, y, n, None, st)
    got = host(y)
    a = O.quantize_act(O.ACT_PER32, x)
    exact, mag = _bound(w_rows, a, k)
    assert np.all(np.abs(got - exact) <= 1e-5 * mag + 1e-6)
    if O.ref_available():
        ok, worst = close(got, O.ref_qmm_gemv(O.Q4_K, w_rows, x, dq.QMM_INT8, paired))
        assert ok, f"worst error ratio {worst:.3g}"
    w.free()
