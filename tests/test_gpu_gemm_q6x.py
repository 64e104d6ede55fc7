"""GPU parity of the Q6_K GEMM on the f16 matrix cores (dq_gemm_q6x.hip) for qmm's two
contracts: per-32 rows (the int8 contract, qmm_reference.cpp:68-93 with Fmt<kQ6_K>) and
int16 rows (ActBlockQ16, kernels_avx2.cpp:1661-1765), through dq_gemm on the block rows,
dq_matmul_act on fp32 rows (which takes it from 3 rows) and dq_qmm_gemm.

The weight w = sc (q - 32) is split exactly into two f16 operands (fh (q - 32) and
fl (q - 32), sc = fh + fl), so the per-block integers are exact (per-32; int16: rounded to
fp32 where a running sum passes 2^24) and the fp32 terms are summed in an order of the
kernel's own. It is held to the
reference's bound against the exact product, |y - y_exact| <= 1e-5 * sum |w_i x_i|
(dynacore/tests/test_int_kernels.cpp:131-147), and against the oracle's order to the
north-star tolerance (per-32: 1e-4 relative, 1e-5 absolute) or to the int16 GEMV's bar
(int16: 2e-6 * sum |w_i x_i|; its terms reach 2^36 and cancel, so a bar relative to
the output does not fit).

Cases: 1, 5, 16 and 32 super-blocks, workgroups of one 32-row activation tile (up to 32
rows) and of two, whole and partial, super-block ranges
(split K, 2 to 16 ranges) and none, a 128-row weight tile past the last row group
(n = 1088), a row range cutting the first and last tiles, bias,
the extreme weights w = 4096 (sc = -128, q = 0) and w = -3968 with codes of +-127
(+-32767), the reference's edge blocks, and both writers' routes, which must agree bit
for bit.

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

FMTS = [O.ACT_PER32, O.ACT_Q16]
MIN_ROWS = 3  # dq_matmul_act's GEMM threshold for Q6_K x per-32 / int16


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint32)


def _bound(fmt: int, w_rows: np.ndarray, a: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    wf = O.dequantize(O.Q6_K, w_rows, k).astype(np.float64)
    af = O.dequantize_act(fmt, a, k).astype(np.float64)
    return af @ wf.T, np.abs(af) @ np.abs(wf).T


def _extreme(w_rows: np.ndarray, n: int, k: int) -> None:
    """Rows 5 i: every scale -128; rows 5 i + 1: also every q = 0 (w = 4096); rows
    5 i + 2: every q = 63 at scale -128 (w = -3968)."""
    b = w_rows.reshape(n, k // 256, 210)
    b[::5, :, 192:208] = 0x80
    b[1::5, :, 0:192] = 0x00
    b[1::5, :, 192:208] = 0x80
    b[2::5, :, 0:192] = 0xFF
    b[2::5, :, 192:208] = 0x80


def _vs_oracle(fmt: int, got: np.ndarray, want: np.ndarray, mag: np.ndarray) -> None:
    if fmt == O.ACT_Q16:
        d = np.abs(got - want.astype(np.float64))
        assert np.all(d <= 2e-6 * mag + 1e-30), f"oracle: worst {np.max(d / (2e-6 * mag + 1e-30)):.3g}"
    else:
        ok, worst = close(got, want)
        assert ok, f"oracle: worst error ratio {worst:.3g}"


def _check(fmt: int, m: int, k: int, n: int, n0: int, n1: int, seed: int, extreme: bool = False,
           stress: bool = False) -> None:
    import dqtorch as T

    if stress:
        w_rows = weight_rows(O.Q6_K, n, k, seed, edge=True)
    else:
        w_rows = gguf_weights(O.Q6_K, n, k, seed, outlier_frac=0.01)
    if extreme:
        _extreme(w_rows, n, k)
    x = activations(m, k, seed + 1, outliers=stress)
    if extreme:
        x[0] = 3.0  # every code 127 (32767)
        x[m - 1] = -3.0
    a = O.quantize_act(fmt, x)
    w = dq.Weight.upload(O.Q6_K, w_rows, k)
    bias = np.linspace(-2.5, 2.5, n, dtype=np.float32)
    ad, bd = dev(a), dev(bias)
    out = torch.full((m, n), 777.0, device="cuda")
    T.gemm(w, fmt, ad, n0=n0, n1=n1, bias=bd, out=out)
    yg = host(out)
    assert np.all(yg[:, :n0] == 777.0) and np.all(yg[:, n1:] == 777.0), "writes outside the row range"
    exact, mag = _bound(fmt, w_rows, a, k)
    exact += bias
    err = np.abs(yg[:, n0:n1] - exact[:, n0:n1])
    assert np.all(err <= 1e-5 * mag[:, n0:n1] + 1e-6), f"worst {np.max(err / (1e-5 * mag[:, n0:n1] + 1e-6)):.3g}"
    if not stress:
        want = O.matmul(O.Q6_K, fmt, w_rows, a, k, bias)
        _vs_oracle(fmt, yg[:, n0:n1], want[:, n0:n1], mag[:, n0:n1])
    if n0 == 0 and n1 == n and m >= MIN_ROWS:
        # fp32 rows: quantized and converted inside dq_matmul_act
        ym = host(T.matmul_act(w, fmt, dev(x), bias=bd))
        assert np.array_equal(bits(ym), bits(yg)), "dq_matmul_act differs from dq_gemm on the same rows"
    w.free()


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m,k", [(5, 256), (16, 256), (67, 1280), (130, 4096), (20, 8192)])
def test_q6x_gemm_superblock_counts(cuda, fmt, m, k):
    """1, 5, 16 and 32 super-blocks; every m ends on a partial activation tile (32 rows up
    to m = 32, else 64). With
    8 weight tiles the super-blocks split into ranges (2 at K=1280, 8 at K=4096, 16 at
    K=8192) whose partials a second launch adds."""
    _check(fmt, m, k, 1024, 0, 1024, 9600 + m + 7 * fmt)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m", [1, 31, 32, 33])
def test_q6x_gemm_tile_rows(cuda, fmt, m):
    """Around the switch from one 32-row activation tile per workgroup (m <= 32) to two:
    one row, a partial and a whole single tile, and a second tile with one row; 8 weight
    tiles, each in 8 super-block ranges."""
    _check(fmt, m, 4096, 1024, 0, 1024, 9650 + m + 7 * fmt)


@pytest.mark.parametrize("fmt", FMTS)
def test_q6x_gemm_tile_past_last_group(cuda, fmt):
    """n = 1088 (17 row groups): the last 128-row weight tile's second group lies past the
    weight, whose loads return zeros and whose outputs are not stored."""
    _check(fmt, 40, 512, 1088, 0, 1088, 9700 + fmt)


@pytest.mark.parametrize("fmt", FMTS)
def test_q6x_gemm_row_range(cuda, fmt):
    """A row range that starts inside the first 64-row group and ends inside the last
    128-row weight tile: whole tiles computed, only [n0, n1) stored."""
    _check(fmt, 80, 1024, 1536, 37, 1500, 9800 + fmt)


@pytest.mark.parametrize("fmt", FMTS)
def test_q6x_gemm_extreme_weights(cuda, fmt):
    """w = 4096 and w = -3968 over whole rows against codes of +-127 (+-32767): the
    largest per-block sums (32 * 4096 * 127 < 2^24 for per-32)."""
    _check(fmt, 72, 512, 1024, 0, 1024, 9900 + fmt, extreme=True)


@pytest.mark.parametrize("fmt", FMTS)
def test_q6x_gemm_stress(cuda, fmt):
    """The reference's edge blocks (d = 0, saturated and negative scales, random bytes)
    with outlier activations, against the exact product."""
    _check(fmt, 72, 512, 1024, 0, 1024, 9950 + fmt, stress=True)


@pytest.mark.parametrize("fmt", FMTS)
def test_q6x_gemm_down_shape(cuda, fmt):
    """Config 3's FFN down shape (K=14336, N=4096) at M=512: 256 tiles, each in two ranges
    of 28 super-blocks (two workgroups per CU); 192 sampled columns against the exact
    product and the oracle."""
    import dqtorch as T

    m, k, n = 512, 14336, 4096
    w_rows = gguf_weights(O.Q6_K, n, k, 9990 + fmt, outlier_frac=0.01)
    x = activations(m, k, 9991 + fmt, outliers=False)
    w = dq.Weight.upload(O.Q6_K, w_rows, k)
    ym = host(T.matmul_act(w, fmt, dev(x)))
    a = O.quantize_act(fmt, x)
    cols = np.random.default_rng(9992).choice(n, 192, replace=False)
    exact, mag = _bound(fmt, w_rows[cols], a, k)
    assert np.all(np.abs(ym[:, cols] - exact) <= 1e-5 * mag)
    _vs_oracle(fmt, ym[:, cols], O.matmul(O.Q6_K, fmt, w_rows[cols], a, k), mag)
    w.free()


@pytest.mark.parametrize("mode", ["int8", "int16"])
@pytest.mark.parametrize("paired", [False, True])
def test_q6x_qmm_gemm(cuda, mode, paired):
    """dq_qmm_gemm on a qmm buffer of 150 rows: the GEMM on the buffer's blocks, within
    tolerance of the reference build's qmm gemv (its own fp32 order)."""
    qm = dq.QMM_INT8 if mode == "int8" else dq.QMM_INT16
    fmt = O.ACT_PER32 if mode == "int8" else O.ACT_Q16
    m, k, n = 150, 1024, 512
    w_rows = gguf_weights(O.Q6_K, n, k, 9995, outlier_frac=0.01)
    x = activations(m, k, 9996, outliers=False)
    w = dq.Weight.upload(O.Q6_K, w_rows, k)
    nbytes = dq.qmm_act_bytes(qm, m, k, paired)
    buf = torch.empty((nbytes,), dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    acts = dq.qmm_act_prepare(buf, nbytes, qm, m, k, paired, st)
    dq.qmm_quantize_rows(dev(x), k, 0, m, acts, st)
    y = torch.zeros((m, n), device="cuda")
    dq.qmm_gemm(w, 0, n, acts, y, n, None, st)
    got = host(y)
    a = O.quantize_act(fmt, x)
    exact, mag = _bound(fmt, w_rows, a, k)
    assert np.all(np.abs(got - exact) <= 1e-5 * mag + 1e-6)
    if O.ref_available():
        _vs_oracle(fmt, got, O.ref_qmm_gemv(O.Q6_K, w_rows, x, qm, paired), mag)
    w.free()
