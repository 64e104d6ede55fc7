"""The fp32 expand + GEMM class on the matrix cores (dq_gemm_f32.hip; dynacore's
kF32ExpandGemm, cpu_device.cpp:1114-1152), reached through dq_matmul_plan with the
default plan at m >= DQ_F32_GEMM_MIN_ROWS for dense rows.

- The expansion is bit-exact: one-hot activation rows read each expanded weight back
  unchanged, and it equals the oracle's x86 expansion (pinned to the reference's own
  in tests/test_expand.py).
- The sums run in the matrix cores' order, so the bar is the class tolerance, 1e-5 of
  sum |x_k w_k|, against the exact fp64 product of the expanded operands, against the
  oracle's vec_dot order and against the reference's own expand + GEMM outputs
  (tests/golden/expand_vectors.npz).
- A row's outputs do not depend on the other rows of the call."""
from __future__ import annotations

import os

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import TYPES, activations, gguf_weights
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
REL = 1e-5  # the class tolerance, relative to sum |x_k w_k|


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def run(w, xd, bias=None):
    """dq_matmul_plan with the default plan on the rows of xd (a 2-D device view)."""
    import dqtorch as T

    m = xd.shape[0]
    y = torch.empty((m, w.n), device="cuda")
    dq.matmul_plan(w, None, xd, m, xd.stride(0), y, y.stride(0), bias, T.stream())
    return host(y)


def bound(t, rows, x, k):
    wx = O.expand_x86(t, rows, k).astype(np.float64)
    xf = np.asarray(x, np.float64)
    return xf @ wx.T, np.abs(xf) @ np.abs(wx).T


def kdim(t):
    return 1280 if t in (O.Q4_K, O.Q6_K) else 1312  # 41 blocks of 32: the last slice is half empty


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_selected_from_min_rows(t):
    k = kdim(t)
    assert dq.select(dq.F32_GEMM_MIN_ROWS, 4096, k, t).kernel == dq.KERNEL_F32_EXPAND_GEMM
    assert dq.select(512, 4096, k, t, x_dense=False).kernel == dq.KERNEL_F32_ROW_DOT


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_expansion_bit_exact_one_hot(cuda, t):
    """x = the identity (K rows): output row k is column k of the expanded weights."""
    k = kdim(t)
    n = 136  # three row groups, the last two in one tile
    rows = gguf_weights(t, n, k, 3100 + t, outlier_frac=0.02)
    y = run(dq.Weight.upload(t, rows, k), dev(np.eye(k, dtype=np.float32)))
    assert np.array_equal(y.T.view(np.uint32), O.expand_x86(t, rows, k).view(np.uint32))


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
@pytest.mark.parametrize("m", [16, 37, 130])
def test_parity(cuda, t, m):
    k = kdim(t)
    n = 200
    rows = gguf_weights(t, n, k, 3200 + t + m, outlier_frac=0.01)
    x = activations(m, k, 3300 + m)
    xs = np.zeros((m, k + 3), np.float32)  # strided rows, read in place
    xs[:, :k] = x
    bias = O.normal(3400 + m, n)
    w = dq.Weight.upload(t, rows, k)
    y = run(w, dev(xs)[:, :k], dev(bias)) - bias  # bias added after the sum
    exact, mag = bound(t, rows, x, k)
    assert np.all(np.abs(y - exact) <= REL * mag + 1e-30)
    want = O.matmul(t, O.ACT_F32, rows, O.quantize_act(O.ACT_F32, x), k)  # the vec_dot order
    assert np.all(np.abs(y - want) <= REL * mag + 1e-30)


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_rows_independent(cuda, t):
    """The first 16 rows give the same bits alone as inside a 130-row call, with a
    bias and without."""
    k = kdim(t)
    rows = gguf_weights(t, 200, k, 3500 + t)
    x = dev(activations(130, k, 3501))
    w = dq.Weight.upload(t, rows, k)
    a, b = run(w, x), run(w, x[:16])
    assert np.array_equal(a[:16].view(np.uint32), b.view(np.uint32))
    bias = dev(O.normal(3502, 200))
    assert np.array_equal(run(w, x, bias)[:16].view(np.uint32), run(w, x[:16], bias).view(np.uint32))


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_reference_golden(cuda, t):
    """The golden rows (K = 512) and the seeded ones (K = 1024 / 1056): within the class
    bound of the reference's own expand + GEMM and of its generic vec_dot (vecdot_*)."""
    ev = np.load(os.path.join(GOLDEN, "expand_vectors.npz"))
    rv = np.load(os.path.join(GOLDEN, "reference_vectors.npz"))
    name = O.TYPE_NAMES[t]
    w_rows, x = rv[f"w_{name}"], rv["act_x"]
    xx = np.tile(x, (5, 1))  # 20 rows: past DQ_F32_GEMM_MIN_ROWS
    y = run(dq.Weight.upload(t, w_rows, 512), dev(xx))
    _, mag = bound(t, w_rows, xx, 512)
    assert np.all(np.abs(y - np.tile(ev[f"expgemm_{name}"], (5, 1))) <= REL * mag)
    assert np.all(np.abs(y - np.tile(rv[f"vecdot_{name}"], (5, 1))) <= REL * mag)
    rw, gx = ev[f"rw_{name}"], ev[f"gx_{name}"]
    k = gx.shape[1]
    y = run(dq.Weight.upload(t, rw, k), dev(gx))
    _, mag = bound(t, rw, gx, k)
    assert np.all(np.abs(y - ev[f"expgemm_rw_{name}"]) <= REL * mag)


def test_bench_shape(cuda):
    """Config 4's prefill shape (Q4_K, K = 4096, N = 14336, M = 512) through the fp32
    class: 192 sampled weight rows against the exact product."""
    k, n, m = 4096, 14336, 512
    rng = np.random.default_rng(3600)  # random valid blocks: any codes and scales, fp16 d / dmin small
    rows = rng.integers(0, 256, (n, k // 256, 144), dtype=np.uint8)
    rows[:, :, 0:4] = rng.uniform(0.002, 0.02, (n, k // 256, 2)).astype(np.float16).view(np.uint8).reshape(n, -1, 4)
    rows = rows.reshape(n, -1)
    x = activations(m, k, 3601)
    y = run(dq.Weight.upload(O.Q4_K, rows, k), dev(x))
    cols = np.random.default_rng(3602).choice(n, 192, replace=False)
    cols.sort()
    exact, mag = bound(O.Q4_K, rows[cols], x, k)
    assert np.all(np.abs(y[:, cols] - exact) <= REL * mag)


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_wide_tiles(cuda, t):
    """A shape whose grid takes the 224-row weight tiles (M = 300, N = 14000: 189 tiles of
    224 rows against 330 of 128), the last tile running past the weight's padded rows:
    every output against the exact product, and the first 16 rows bit-equal alone."""
    k = 256 if t in (O.Q4_K, O.Q6_K) else 96
    n, m = 14000, 300
    rows = gguf_weights(t, n, k, 3700 + t)
    x = activations(m, k, 3701)
    w = dq.Weight.upload(t, rows, k)
    xd = dev(x)
    y = run(w, xd)
    exact, mag = bound(t, rows, x, k)
    assert np.all(np.abs(y - exact) <= REL * mag + 1e-30)
    assert np.array_equal(y[:16].view(np.uint32), run(w, xd[:16]).view(np.uint32))
