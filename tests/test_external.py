"""The host-memory adapter (dq_external_*): dynacore's ExternalMatmulKernel shape
{eligible(shape, weight), run(x, w, bias, y)} (dynacore/include/dynacore/cpu/cpu_device.h:22-30)
over host arrays, with device copies of the weights kept across calls.

The reference's own test of the extension point (dynacore/tests/test_matmul_registry.cpp:679-728)
checks that eligibility is a pure shape rule and that run's results match a double
reference within 1e-6; here run must equal dq_matmul_plan under the adapter's plan (the
defaults unless set) on the same rows bit for bit, and the oracle under the selected
activation contract within the fp32 bar. Eligibility needs no GPU and runs on the CPU.
"""
from __future__ import annotations

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import TYPES, activations, close, gguf_weights
from oracle import oracle as O


def _shape(m, n, k, t, dense=1):
    return dq.MatmulShape(m, n, k, t, dense)


def test_eligible_is_a_shape_rule():
    """validate_matmul_shape's rules (dynacore/src/kernel/matmul_registry.cpp:264-278) for the
    four weight types; no tensor data is read (a dummy weight address serves)."""
    w = 0x1000
    assert dq.external_eligible(_shape(1, 4096, 4096, dq.Q4_K), w)
    assert dq.external_eligible(_shape(512, 14336, 4096, dq.Q4_K, 0), w)
    assert dq.external_eligible(_shape(7, 256, 512, dq.Q8_0), w)
    assert dq.external_eligible(_shape(3, 96, 64, dq.Q4_0), w)
    assert dq.external_eligible(_shape(2, 10, 14336, dq.Q6_K), w)
    assert not dq.external_eligible(_shape(1, 4096, 4000, dq.Q4_K), w)     # k not a whole number of blocks
    assert not dq.external_eligible(_shape(0, 4096, 4096, dq.Q4_K), w)     # empty
    assert not dq.external_eligible(_shape(1, 0, 4096, dq.Q4_K), w)
    assert not dq.external_eligible(_shape(1, 4096, 4096, 1), w)           # fp16 weights: not this library's
    assert not dq.external_eligible(_shape(1, 4096, 4096, dq.Q4_K), 0)     # no weight


# ------------------------------------------------------------------------- GPU


def _torch():
    return pytest.importorskip("torch")


def _dq_matmul(t, rows, k, x, bias, plan=None):
    """dq_matmul_plan on device copies of the same rows (the path run() wraps)."""
    torch = _torch()
    import dqtorch as T

    w = dq.Weight.upload(t, rows, k)
    if x.strides[0] != 4 * k:
        # a view of wider rows: keep the caller's row stride on the device (the layout
        # decides between the fp32 expand and row kernels)
        xd = torch.from_numpy(np.ascontiguousarray(x.base)).cuda()[:, :k]
    else:
        xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    bd = torch.from_numpy(bias).cuda() if bias is not None else None
    y = torch.empty((x.shape[0], w.n), device="cuda")
    dq.matmul_plan(w, plan, xd, x.shape[0], xd.stride(0), y, y.stride(0), bd, T.stream())
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
@pytest.mark.parametrize("m", [1, 5, 40, 130])
def test_run_equals_dq_matmul(cuda, t, m):
    """Strided host x, padded weight rows, a bias and a strided y: the same bits as
    dq_matmul on the device, and within the fp32 bar of the oracle."""
    k, n = 1024, 200
    rows = gguf_weights(t, n, k, 1700 + t + m, outlier_frac=0.01)
    padded = np.zeros((n, rows.shape[1] + 16), np.uint8)
    padded[:, :rows.shape[1]] = rows
    x = activations(m, k, 1710 + m)
    xs = np.zeros((m, k + 9), np.float32)
    xs[:, :k] = x
    bias = O.normal(1720 + m, n)
    ybuf = np.full((m, n + 3), np.nan, np.float32)
    ad = dq.External(0)
    ad.run(xs[:, :k], padded, t, k, bias=bias, y=ybuf[:, :n])
    assert np.isnan(ybuf[:, n:]).all()
    y = ybuf[:, :n]
    want = _dq_matmul(t, rows, k, xs[:, :k], bias)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
    # the selection is made on the caller's layout of x (strided here)
    fmt = dq.select(m, n, k, t, x_dense=m == 1).act
    ok, worst = close(y, O.matmul(t, fmt, rows, O.quantize_act(fmt, x), k, bias=bias))
    assert ok, worst
    st = ad.stats()
    assert st["runs"] == 1 and st["uploads"] == 1 and st["resident_weights"] == 1
    ad.close()


@pytest.mark.gpu
def test_weight_copies_are_kept_and_evicted(cuda):
    """One device copy per host weight: a second run finds it; with a byte limit of
    one copy the least recently used copy is dropped; forget() drops a copy."""
    k, n = 512, 256
    wa = gguf_weights(O.Q4_K, n, k, 1800)
    wb = gguf_weights(O.Q4_K, n, k, 1801)
    x = activations(3, k, 1802)
    one = (n + 63) // 64 * 64 * O.row_bytes(O.Q4_K, k)
    ad = dq.External(0, max_resident_bytes=one + 100)
    ya = ad.run(x, wa, dq.Q4_K, k)
    assert np.array_equal(ad.run(x, wa, dq.Q4_K, k), ya)
    st = ad.stats()
    assert (st["uploads"], st["hits"], st["evictions"], st["resident_bytes"]) == (1, 1, 0, one)
    yb = ad.run(x, wb, dq.Q4_K, k)
    assert ad.stats()["evictions"] == 1 and ad.stats()["resident_weights"] == 1
    assert np.array_equal(ad.run(x, wa, dq.Q4_K, k), ya)       # uploaded again
    st = ad.stats()
    assert (st["runs"], st["uploads"], st["hits"], st["evictions"]) == (4, 3, 1, 2)
    assert np.array_equal(yb, _dq_matmul(O.Q4_K, wb, k, x, None))
    ad.forget(wa)
    assert ad.stats()["resident_weights"] == 0 and ad.stats()["resident_bytes"] == 0
    with pytest.raises(dq.DqError) as e:
        ad.forget(wa)
    assert e.value.status == "not_found"
    ad.close()


@pytest.mark.gpu
def test_weight_over_the_limit_is_not_kept(cuda):
    k, n = 512, 256
    w = gguf_weights(O.Q6_K, n, k, 1900)
    x = activations(2, k, 1901)
    ad = dq.External(0, max_resident_bytes=1024)
    y = ad.run(x, w, dq.Q6_K, k)
    st = ad.stats()
    assert st["uploads"] == 1 and st["resident_weights"] == 0 and st["resident_bytes"] == 0
    assert np.array_equal(y, _dq_matmul(O.Q6_K, w, k, x, None))
    ad.close()


@pytest.mark.gpu
def test_min_rows_policy_and_rejected_calls(cuda):
    """eligible() applies the adapter's row floor (the caller's choice of which calls go
    to the GPU, as the reference's test kernel takes only m == 7); run() rejects bad
    arguments with dynacore status codes before any copy."""
    ad = dq.External(0, min_rows=9)
    w = 0x1000
    assert not ad.eligible(8, 4096, 4096, dq.Q4_K, w)
    assert ad.eligible(9, 4096, 4096, dq.Q4_K, w)
    x = np.zeros((2, 256), np.float32)
    rows = np.zeros((4, O.row_bytes(O.Q4_K, 256)), np.uint8)
    with pytest.raises(dq.DqError) as e:
        ad.run(x, rows, 1, 256)
    assert e.value.status == "unsupported"
    with pytest.raises(dq.DqError) as e:
        ad.run(x[:, :200], rows, dq.Q4_K, 200)
    assert e.value.status == "invalid_argument"
    with pytest.raises(dq.DqError) as e:
        dq.External(0, min_rows=0)
    assert e.value.status == "invalid_argument"
    assert ad.stats()["runs"] == 0
    ad.close()


@pytest.mark.gpu
def test_set_plan_selects_the_contract(cuda):
    """Device::set_kernel_plan: the defaults (qmm on: qmm's gemv on per-32 rows at 4
    rows); without qmm the sub-scaled class; the FFN down plan moves a Q6_K decode call
    to int16 activations; the all-integer plan reproduces dq_matmul (the super-block
    class) bit for bit; NULL restores the defaults."""
    torch = _torch()
    import dqtorch as T

    k, n, m = 1536, 256, 4
    rows = gguf_weights(O.Q6_K, n, k, 2000, outlier_frac=0.01)
    x = activations(m, k, 2001)
    x[:, 5::61] *= np.float32(50.0)  # outlier channels, as the down projection's input has
    wd = O.dequantize(O.Q6_K, rows, k).astype(np.float64).reshape(n, k)

    def mag_of(fmt):
        xa = O.dequantize_act(fmt, O.quantize_act(fmt, x), k).astype(np.float64)
        return np.abs(xa) @ np.abs(wd).T

    ad = dq.External(0)
    assert dq.select(m, n, k, dq.Q6_K).kernel == dq.KERNEL_QMM_GEMV
    y_def = ad.run(x, rows, dq.Q6_K, k)
    assert np.array_equal(y_def.view(np.uint32), _dq_matmul(O.Q6_K, rows, k, x, None).view(np.uint32))
    want32 = O.matmul(O.Q6_K, O.ACT_PER32, rows, O.quantize_act(O.ACT_PER32, x), k)
    assert np.all(np.abs(y_def - want32) <= 2e-6 * mag_of(O.ACT_PER32) + 1e-30)
    noqmm = dq.plan_defaults()
    noqmm.qmm = 0
    ad.set_plan(noqmm)
    y_sx = ad.run(x, rows, dq.Q6_K, k)
    assert np.array_equal(y_sx.view(np.uint32),
                          O.matmul(O.Q6_K, O.ACT_SX, rows, O.quantize_act(O.ACT_SX, x), k).view(np.uint32))
    down = dq.plan_ffn_down()
    ad.set_plan(down)
    y16 = ad.run(x, rows, dq.Q6_K, k)
    assert np.array_equal(y16.view(np.uint32), _dq_matmul(O.Q6_K, rows, k, x, None, down).view(np.uint32))
    want16 = O.matmul(O.Q6_K, O.ACT_Q16, rows, O.quantize_act(O.ACT_Q16, x), k)
    assert np.all(np.abs(y16 - want16) <= 2e-6 * mag_of(O.ACT_Q16) + 1e-30)
    allint = dq.Plan(2, 1 << 30, 0, 1, 1 << 30, 0, 0)
    ad.set_plan(allint)
    yq = ad.run(x, rows, dq.Q6_K, k)
    w = dq.Weight.upload(O.Q6_K, rows, k)
    ref = T.matmul(w, torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(yq.view(np.uint32), ref.cpu().numpy().view(np.uint32))
    ad.set_plan(None)
    assert np.array_equal(ad.run(x, rows, dq.Q6_K, k).view(np.uint32), y_def.view(np.uint32))
    ad.close()


@pytest.mark.gpu
def test_two_adapters_do_not_share_scratch(cuda):
    """Each adapter keeps its own temporaries: two adapters run from two threads at once
    (their own streams, different shapes and plans) give the bits of running alone."""
    import threading

    k = 4096
    wa = gguf_weights(O.Q8_0, 1024, k, 2100)
    wb = gguf_weights(O.Q4_K, 768, k, 2101)
    xa = activations(40, k, 2102)
    xb = activations(3, k, 2103)
    a, b = dq.External(0), dq.External(0)
    b.set_plan(dq.Plan(2, 1 << 30, 0, 1, 1 << 30, 0, 0))  # Q8_K: quantize + skinny GEMV
    want_a, want_b = a.run(xa, wa, dq.Q8_0, k), b.run(xb, wb, dq.Q4_K, k)
    errors = []

    def loop(ad, x, w, t, want):
        try:
            for _ in range(25):
                if not np.array_equal(ad.run(x, w, t, k).view(np.uint32), want.view(np.uint32)):
                    errors.append(t)
                    return
        except Exception as e:  # noqa: BLE001 -- reported below
            errors.append(repr(e))

    th = [threading.Thread(target=loop, args=(a, xa, wa, dq.Q8_0, want_a)),
          threading.Thread(target=loop, args=(b, xb, wb, dq.Q4_K, want_b))]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errors, errors
    a.close()
    b.close()
