"""qmm's activation buffer on the GPU (dq_qmm_act_prepare / dq_qmm_quantize_rows) against
the oracle's restatement of ActBuffer + quantize_row_ref (dynacore/cpu/qmm/qmm_reference.cpp:
25-51,440-488), byte for byte; the oracle is pinned to the reference build in test_oracle.py.
Cases follow dynacore/tests/test_qmm.cpp's: both modes and layouts, odd m (pad row), split
row ranges, strided rows, and NaN / Inf / zero / tie inputs."""
from __future__ import annotations

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import TYPES, activations, close, gguf_weights
from oracle import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def rows(m: int, k: int, seed: int) -> np.ndarray:
    x = (np.random.default_rng(seed).standard_normal((m, k)) * 3).astype(np.float32)
    x[0, 3] = np.nan
    x[m - 1, min(40, k - 1)] = np.inf
    if k >= 128:
        x[0, 64:96] = 0.0
        x[0, 96:128] = -0.0
        x[m - 1, 0] = -np.inf
    if k >= 64:
        x[m - 1, 32] = 127.0
        x[m - 1, 33:64] = np.float32(0.5) + np.arange(31, dtype=np.float32)
    return x


def run_gpu(x: np.ndarray, mode: int, paired: bool, x_stride: int | None = None, splits=()):
    """Quantize the rows of x on the GPU (over the row ranges cut at `splits`); return the
    buffer's regions as the oracle returns them."""
    m, k = x.shape
    xs = x_stride or k
    xp = np.zeros((m, xs), np.float32)
    xp[:, :k] = x
    xd = torch.from_numpy(xp).cuda()
    nbytes = dq.qmm_act_bytes(mode, m, k, paired)
    buf = torch.full((nbytes,), 0xAB, dtype=torch.uint8, device="cuda")  # stale contents
    st = torch.cuda.current_stream().cuda_stream
    a = dq.qmm_act_prepare(buf, nbytes, mode, m, k, paired, st)
    cuts = [0, *splits, m]
    for r0, r1 in zip(cuts[:-1], cuts[1:]):
        dq.qmm_quantize_rows(xd, xs, r0, r1, a, st)
    torch.cuda.synchronize()
    h = buf.cpu().numpy()
    base = buf.data_ptr()
    m_pad = (m + 1) // 2 * 2 if paired else m
    ncode, nsc = m_pad * k, m_pad * (k // 32)
    hi = h[a.hi - base:a.hi - base + ncode].view(np.int8)
    lo = h[a.lo - base:a.lo - base + ncode] if mode == 1 else None
    d = h[a.d - base:a.d - base + 4 * nsc].view(np.float32)
    c = h[a.c - base:a.c - base + 4 * nsc].view(np.float32)
    return hi, lo, d, c


def same(got, want):
    for g, w in zip(got, want):
        assert (g is None) == (w is None)
        if g is not None:
            assert g.tobytes() == w.tobytes()


@pytest.mark.parametrize("mode", [dq.QMM_INT8, dq.QMM_INT16])
@pytest.mark.parametrize("paired", [False, True])
@pytest.mark.parametrize("m,k", [(1, 32), (2, 256), (7, 1536), (16, 4096)])
def test_qmm_quantize_bit_exact(cuda, mode, paired, m, k):
    x = rows(m, k, 3 * m + k)
    same(run_gpu(x, mode, paired), O.qmm_quantize(x, mode, paired))


@pytest.mark.parametrize("mode", [dq.QMM_INT8, dq.QMM_INT16])
@pytest.mark.parametrize("paired", [False, True])
def test_qmm_quantize_split_rows_and_stride(cuda, mode, paired):
    """Row ranges quantized by separate calls (odd cut points, so a pair is written by two
    calls) and rows x_stride > k floats apart give the one-call bytes."""
    x = rows(9, 512, 17)
    want = O.qmm_quantize(x, mode, paired)
    same(run_gpu(x, mode, paired, x_stride=544, splits=(3, 4, 7)), want)


@pytest.mark.parametrize("mode", [dq.QMM_INT8, dq.QMM_INT16])
def test_qmm_quantize_prefill_shape(cuda, mode):
    """Config 4's prefill activations (512 rows of 4096) in the gemm's pair layout."""
    x = np.random.default_rng(4).standard_normal((512, 4096)).astype(np.float32)
    same(run_gpu(x, mode, True), O.qmm_quantize(x, mode, True))


def prepared(x: np.ndarray, mode: int, paired: bool):
    m, k = x.shape
    nbytes = dq.qmm_act_bytes(mode, m, k, paired)
    buf = torch.empty((nbytes,), dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    a = dq.qmm_act_prepare(buf, nbytes, mode, m, k, paired, st)
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    dq.qmm_quantize_rows(xd, k, 0, m, a, st)
    return buf, xd, a


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("mode", [dq.QMM_INT8, dq.QMM_INT16])
@pytest.mark.parametrize("paired", [False, True])
def test_qmm_gemv(cuda, t, mode, paired):
    """qmm::Kernels::gemv on the qmm buffer: rows [r0, r0 + rows) of either layout equal
    dq_gemv on the same rows quantized to the per-32 / int16 block format bit for bit, and
    qmm's reference gemv (its own fp32 order) within the north-star tolerance."""
    import dqtorch as T

    m, k, n, r0, rows = 7, 1024, 96, 2, 5
    w_rows = gguf_weights(t, n, k, 31 + t, outlier_frac=0.01)
    x = activations(m, k, 7 * t + mode, outliers=False)
    w = dq.Weight.upload(t, w_rows, k)
    buf, xd, a = prepared(x, mode, paired)
    bias = torch.from_numpy(np.linspace(-1, 1, n, dtype=np.float32)).cuda()
    y = torch.full((m, n), 7.0, device="cuda")
    dq.qmm_gemv(w, 0, n, a, r0, rows, y, n, bias, torch.cuda.current_stream().cuda_stream)
    fmt = O.ACT_PER32 if mode == dq.QMM_INT8 else O.ACT_Q16
    acts = T.quantize(fmt, xd)
    want = T.gemv(w, fmt, acts, bias=bias)
    got = y.cpu().numpy()
    assert np.array_equal(got[r0:r0 + rows].view(np.uint32), want.cpu().numpy()[r0:r0 + rows].view(np.uint32))
    assert (got[:r0] == 7.0).all() and (got[r0 + rows:] == 7.0).all()
    if O.ref_available():
        ref = O.ref_qmm_gemv(t, w_rows, x, mode, paired) + np.linspace(-1, 1, n, dtype=np.float32)
        ok, worst = close(got[r0:r0 + rows], ref[r0:r0 + rows])
        assert ok, f"worst error ratio {worst:.3g}"
    w.free()


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_0, O.Q4_K])
def test_qmm_gemm(cuda, t):
    """qmm::Kernels::gemm on a paired buffer of odd m: every row equals dq_gemm on the
    per-32 rows bit for bit (Q8_0 / Q4_0 on the per-32 int8 MFMA GEMM, Q4_K on the f16
    GEMM, which takes more than 64 rows)."""
    import dqtorch as T

    m, k, n = 67, 2048, 256
    w_rows = gguf_weights(t, n, k, 77 + t, outlier_frac=0.01)
    x = activations(m, k, 5 + t, outliers=False)
    w = dq.Weight.upload(t, w_rows, k)
    buf, xd, a = prepared(x, dq.QMM_INT8, True)
    y = torch.zeros((m, n), device="cuda")
    dq.qmm_gemm(w, 0, n, a, y, n, None, torch.cuda.current_stream().cuda_stream)
    acts = T.quantize(O.ACT_PER32, xd)
    want = T.gemm(w, O.ACT_PER32, acts)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32))
    ok, worst = close(y.cpu().numpy(), O.matmul(t, O.ACT_PER32, w_rows, O.quantize_act(O.ACT_PER32, x), k))
    assert ok, f"worst error ratio {worst:.3g}"
    w.free()


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("mode", [dq.QMM_INT8, dq.QMM_INT16])
def test_qmm_gemv_unaligned_ranges(cuda, t, mode):
    """Callers split [n0, n1) across threads (qmm.h:35-36): three pieces that start and
    end inside 64-row groups give the one-call bits, and a single piece leaves every
    output outside it untouched."""
    m, k, n = 5, 1024, 200
    w_rows = gguf_weights(t, n, k, 91 + t, outlier_frac=0.01)
    x = activations(m, k, 92 + mode, outliers=False)
    w = dq.Weight.upload(t, w_rows, k)
    buf, xd, a = prepared(x, mode, True)
    st = torch.cuda.current_stream().cuda_stream
    full = torch.full((m, n), 7.0, device="cuda")
    dq.qmm_gemv(w, 0, n, a, 0, m, full, n, None, st)
    part = torch.full((m, n), 7.0, device="cuda")
    for n0, n1 in ((0, 37), (37, 150), (150, n)):
        dq.qmm_gemv(w, n0, n1, a, 0, m, part, n, None, st)
    assert np.array_equal(part.cpu().numpy().view(np.uint32), full.cpu().numpy().view(np.uint32))
    one = torch.full((m, n), 7.0, device="cuda")
    dq.qmm_gemv(w, 37, 150, a, 1, 3, one, n, None, st)
    got, ref = one.cpu().numpy(), full.cpu().numpy()
    assert np.array_equal(got[1:4, 37:150].view(np.uint32), ref[1:4, 37:150].view(np.uint32))
    inside = np.zeros_like(got, dtype=bool)
    inside[1:4, 37:150] = True
    assert (got[~inside] == 7.0).all()
    w.free()


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("mode", [dq.QMM_INT8, dq.QMM_INT16])
def test_qmm_gemm_modes_and_ranges(cuda, t, mode):
    """qmm::Kernels::gemm in both modes on every format (int16, Q6_K and small row
    counts run the GEMV passes; Q8_0 / Q4_0 / Q4_K in int8 mode the GEMMs): within the
    north-star tolerance of qmm's reference gemv, and three unaligned [n0, n1) pieces
    give the one-call bits."""
    m, k, n = 67, 1024, 200
    w_rows = gguf_weights(t, n, k, 95 + t, outlier_frac=0.01)
    x = activations(m, k, 96 + mode, outliers=False)
    w = dq.Weight.upload(t, w_rows, k)
    buf, xd, a = prepared(x, mode, True)
    st = torch.cuda.current_stream().cuda_stream
    full = torch.full((m, n), 7.0, device="cuda")
    dq.qmm_gemm(w, 0, n, a, full, n, None, st)
    part = torch.full((m, n), 7.0, device="cuda")
    for n0, n1 in ((0, 37), (37, 150), (150, n)):
        dq.qmm_gemm(w, n0, n1, a, part, n, None, st)
    got = full.cpu().numpy()
    assert np.array_equal(part.cpu().numpy().view(np.uint32), got.view(np.uint32))
    if O.ref_available():
        ok, worst = close(got, O.ref_qmm_gemv(t, w_rows, x, mode, True))
        assert ok, f"worst error ratio {worst:.3g}"
    else:
        fmt = O.ACT_PER32 if mode == dq.QMM_INT8 else O.ACT_Q16
        ok, worst = close(got, O.matmul(t, fmt, w_rows, O.quantize_act(fmt, x), k))
        assert ok, f"worst error ratio {worst:.3g}"
    w.free()
