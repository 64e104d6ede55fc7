"""dq_matmul_plan on the GPU: Device::matmul under a KernelPlan. Each call runs the
kernel dq_select picks (the reference's select_matmul over this library's kernels;
tests/test_plan.py pins the selection itself), with the bits of that contract's path
(dq_matmul_act, or dq_matmul for the integer classes it covers) and the oracle's
result under that contract within the parity bar of each class."""
from __future__ import annotations

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import TYPES, activations, close, gguf_weights
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

ALL_INT8 = dq.Plan(2, 1 << 30, 0, 1, 1 << 30, 0, 0)  # dq_matmul's plan: super-block / per-32 at every m


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def within_terms(y, want, t, fmt, rows, x, k, rel=2e-6):
    """|y - want| <= rel * sum_k |x_k w_k| (the reference's bound form,
    dynacore/tests/test_int_kernels.cpp:181-193), on the dequantized operands."""
    xa = x.astype(np.float64) if fmt == O.ACT_F32 else O.dequantize_act(fmt, O.quantize_act(fmt, x), k).astype(
        np.float64)
    wd = O.dequantize(t, rows, k).astype(np.float64).reshape(rows.shape[0], k)
    mag = np.abs(xa) @ np.abs(wd).T
    return bool(np.all(np.abs(y.astype(np.float64) - want) <= rel * mag + 1e-30))


def run_plan(w, plan, x, bias=None):
    import dqtorch as T

    xd = dev(x) if isinstance(x, np.ndarray) else x
    y = torch.empty((xd.shape[0], w.n), device="cuda")
    dq.matmul_plan(w, plan, xd, xd.shape[0], xd.stride(0), y, y.stride(0), bias, T.stream())
    return host(y)


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
@pytest.mark.parametrize("m", [1, 3, 4, 5, 8, 9, 40])
def test_default_plan(cuda, t, m):
    import dqtorch as T

    k, n = 1536, 200
    rows = gguf_weights(t, n, k, 2200 + t + m, outlier_frac=0.01)
    x = activations(m, k, 2201 + m)
    w = dq.Weight.upload(t, rows, k)
    sel = dq.select(m, n, k, t)
    y = run_plan(w, None, x)
    # the same bits as the selected contract's own path
    mfma_f32 = sel.kernel == dq.KERNEL_F32_EXPAND_GEMM and m >= dq.F32_GEMM_MIN_ROWS
    if sel.kernel == dq.KERNEL_INT8_PER32 and t in (O.Q8_0, O.Q4_0):
        same = host(T.matmul(w, dev(x)))
    elif not mfma_f32:  # the matrix-core GEMM sums in its own order (tests/test_gpu_f32_gemm.py)
        same = host(T.matmul_act(w, sel.act, dev(x)))
    if not mfma_f32:
        assert np.array_equal(y.view(np.uint32), same.view(np.uint32)), dq.KERNEL_NAMES[sel.kernel]
    want = O.matmul(t, sel.act, rows, O.quantize_act(sel.act, x), k)
    if sel.act == O.ACT_SX:
        assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
    elif sel.act == O.ACT_PER32:
        ok, worst = close(y, want)
        assert ok, f"{dq.KERNEL_NAMES[sel.kernel]}: worst error ratio {worst:.3g}"
    else:
        assert within_terms(y, want, t, sel.act, rows, x, k, rel=1e-5 if mfma_f32 else 2e-6), dq.KERNEL_NAMES[sel.kernel]


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
@pytest.mark.parametrize("m", [1, 5, 40, 300])
def test_all_int8_plan_is_dq_matmul(cuda, t, m):
    import dqtorch as T

    k, n = 1024, 256
    rows = gguf_weights(t, n, k, 2300 + t + m)
    x = activations(m, k, 2301 + m)
    w = dq.Weight.upload(t, rows, k)
    assert np.array_equal(run_plan(w, ALL_INT8, x).view(np.uint32), host(T.matmul(w, dev(x))).view(np.uint32))


@pytest.mark.parametrize("t", [O.Q6_K, O.Q4_K, O.Q8_0, O.Q4_0], ids=lambda t: O.TYPE_NAMES[t])
def test_ffn_down_plan_int16(cuda, t):
    """The down projection's plan: int16 activations up to 8 rows at K = 14336."""
    import dqtorch as T

    k, n, m = 14336, 256, 6
    rows = gguf_weights(t, n, k, 2400 + t)
    x = activations(m, k, 2401)
    x[:, 11::97] *= np.float32(60.0)
    w = dq.Weight.upload(t, rows, k)
    down = dq.plan_ffn_down()
    assert dq.select(m, n, k, t, down).act == O.ACT_Q16
    y = run_plan(w, down, x)
    assert np.array_equal(y.view(np.uint32), host(T.matmul_act(w, O.ACT_Q16, dev(x))).view(np.uint32))
    assert within_terms(y, O.matmul(t, O.ACT_Q16, rows, O.quantize_act(O.ACT_Q16, x), k), t, O.ACT_Q16, rows, x, k)


@pytest.mark.parametrize("t,m", [(O.Q4_K, 300), (O.Q4_K, 40), (O.Q8_0, 130), (O.Q6_K, 70)],
                         ids=["q4_K-300", "q4_K-40", "q8_0-130", "q6_K-70"])
def test_engine_qmm_plan(cuda, t, m):
    """The engine's plan on a backend with accelerated qmm (int8 rows unbounded,
    dynalm/src/runtime/engine.cpp:365-375): qmm's gemm on per-32 rows from 9 rows (Q4_K:
    the f16 GEMM above 64 rows, Q6_K: from 3 rows, GEMV passes below); the same bits as
    the per-32 contract's own path, within tolerance of the oracle."""
    import dqtorch as T

    k, n = 1024, 512
    rows = gguf_weights(t, n, k, 2600 + t + m, outlier_frac=0.01)
    x = activations(m, k, 2601 + m, outliers=False)
    w = dq.Weight.upload(t, rows, k)
    eng = dq.plan_defaults()
    eng.int8_decode_max_rows = 1 << 30
    sel = dq.select(m, n, k, t, eng)
    assert (sel.kernel, sel.act) == (dq.KERNEL_QMM_GEMM, O.ACT_PER32)
    y = run_plan(w, eng, x)
    assert np.array_equal(y.view(np.uint32), host(T.matmul_act(w, O.ACT_PER32, dev(x))).view(np.uint32))
    ok, worst = close(y, O.matmul(t, O.ACT_PER32, rows, O.quantize_act(O.ACT_PER32, x), k))
    assert ok, f"worst error ratio {worst:.3g}"


def test_strided_rows_select_the_row_kernel(cuda):
    """x_dense comes from the caller's row stride: strided fp32 rows take f32_row_dot,
    dense ones f32_expand_gemm; both are the fp32 contract."""
    k, n, m = 1024, 128, 12
    rows = gguf_weights(O.Q4_0, n, k, 2500)
    x = activations(m, k, 2501)
    xs = np.zeros((m, k + 7), np.float32)
    xs[:, :k] = x
    w = dq.Weight.upload(O.Q4_0, rows, k)
    assert dq.select(m, n, k, O.Q4_0, x_dense=False).kernel == dq.KERNEL_F32_ROW_DOT
    y_strided = run_plan(w, None, dev(xs)[:, :k])
    y_dense = run_plan(w, None, x)
    want = O.matmul(O.Q4_0, O.ACT_F32, rows, O.quantize_act(O.ACT_F32, x), k)
    for y in (y_strided, y_dense):
        assert within_terms(y, want, O.Q4_0, O.ACT_F32, rows, x, k)
