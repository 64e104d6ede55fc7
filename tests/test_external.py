"""The host-memory adapter (dq_external_*): dynacore's ExternalMatmulKernel shape
{eligible(shape, weight), run(x, w, bias, y)} (dynacore/include/dynacore/cpu/cpu_device.h:22-30)
over host arrays, with device copies of the weights kept across calls.

The reference's own test of the extension point (dynacore/tests/test_matmul_registry.cpp:679-728)
checks that eligibility is a pure shape rule and that run's results match a double
reference within 1e-6; here run must equal dq_matmul on the same rows bit for bit, and
the oracle within the fp32 bar. Eligibility needs no GPU and runs on the CPU.
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


def _dq_matmul(t, rows, k, x, bias):
    """dq_matmul on device copies of the same rows (the path run() wraps)."""
    torch = _torch()
    from dynalm_amd import torch_ops as T

    w = dq.Weight.upload(t, rows, k)
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    bd = torch.from_numpy(bias).cuda() if bias is not None else None
    y = T.matmul(w, xd, bd)
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
    want = _dq_matmul(t, rows, k, x, bias)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
    fmt = O.ACT_Q8_K if t in (O.Q4_K, O.Q6_K) else O.ACT_PER32
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
