"""GPU parity of the one-row Q4_K x Q8_K decode launch on 56-row workgroups
(k_gemv_slab, dq_gemv.hip), which dq_gemv / dq_matmul take at M = 1 for rows of
2048 or 4096 values when the weight has at most 56/64 as many row groups as the
GPU has CUs (config 3's gate shape: 256 workgroups instead of 224).

Bar: bit-equal to the oracle (the Q8_K pair's integer S, Mn and canonical fp32
steps) and to the 64-row-group launch that an M = 2 pass takes on the same rows,
with the integer partials S / Mn through dq_debug_partials bit-exact. The cases
cover row counts that end inside a 56-row workgroup and inside a 64-row group, row
ranges cutting workgroup and group boundaries, bias, the reference's edge blocks,
and the fused path (fp32 row quantized in the kernel) against quantize + GEMV.

Reference style: dynacore/tests/test_qmm.cpp:178-282 (odd shapes, split ranges).
"""
from __future__ import annotations

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import activations, weight_rows
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


@pytest.mark.parametrize("k", [2048, 4096])
@pytest.mark.parametrize("n", [50, 120, 1000])
def test_slab_equals_oracle_and_row_groups(cuda, k, n):
    import dqtorch as T

    w_rows = weight_rows(O.Q4_K, n, k, 7000 + n, edge=True)
    x = activations(2, k, 7001 + n)
    a = O.quantize_act(O.ACT_Q8_K, x)
    w = dq.Weight.upload(O.Q4_K, w_rows, k)
    bias = np.linspace(-3.0, 3.0, n, dtype=np.float32)
    ad, bd = dev(a), dev(bias)
    y1 = host(T.gemv(w, O.ACT_Q8_K, ad[:1], bias=bd))
    y2 = host(T.gemv(w, O.ACT_Q8_K, ad, bias=bd))  # two rows: one workgroup per 64-row group
    want = O.matmul(O.Q4_K, O.ACT_Q8_K, w_rows, a[:1], k, bias)
    assert np.array_equal(bits(y1), bits(want))
    assert np.array_equal(bits(y1[0]), bits(y2[0]))
    yf = host(T.matmul(w, dev(x[:1]), bias=bd))  # fused: quantized inside the launch
    assert np.array_equal(bits(yf), bits(y1))
    w.free()


@pytest.mark.parametrize("n0,n1", [(13, 41), (55, 57), (56, 112), (63, 65), (100, 999), (0, 1000), (930, 1000)])
def test_slab_row_ranges(cuda, n0, n1):
    """Rows [n0, n1) only (qmm.h:35-36 ranges): untouched outside, equal to the full call
    inside, for ranges that start and end inside 56-row workgroups and 64-row groups
    (the launch starts at the 64-row group holding n0)."""
    import dqtorch as T

    k, n = 4096, 1000
    w_rows = weight_rows(O.Q4_K, n, k, 7100)
    x = dev(activations(1, k, 7101))
    a = T.quantize(O.ACT_Q8_K, x)
    w = dq.Weight.upload(O.Q4_K, w_rows, k)
    full = host(T.gemv(w, O.ACT_Q8_K, a))
    out = torch.full((1, n), 777.0, device="cuda")
    T.gemv(w, O.ACT_Q8_K, a, n0=n0, n1=n1, out=out)
    part = host(out)
    assert np.all(part[:, :n0] == 777.0) and np.all(part[:, n1:] == 777.0)
    assert np.array_equal(bits(part[:, n0:n1]), bits(full[:, n0:n1]))
    w.free()


def test_slab_partials(cuda):
    """dq_debug_partials at M = 1 through the slab launch: S and Mn per row and
    super-block bit-exact against the oracle."""
    import dqtorch as T

    k, n = 2048, 130
    w_rows = weight_rows(O.Q4_K, n, k, 7200, edge=True)
    a = O.quantize_act(O.ACT_Q8_K, activations(1, k, 7201))
    w = dq.Weight.upload(O.Q4_K, w_rows, k)
    units, sb = T.partials(w, O.ACT_Q8_K, dev(a))
    want_u, want_sb = O.partials(O.Q4_K, O.ACT_Q8_K, w_rows, a, k)
    assert np.array_equal(host(units), want_u)
    assert np.array_equal(host(sb), want_sb)
    w.free()


def test_slab_config3_shape(cuda):
    """Config 3's gate shape (K = 4096, N = 14336): 256 workgroups. Every row equals
    the 64-row-group launch of an M = 2 pass; sampled rows equal the oracle."""
    import dqtorch as T

    k, n = 4096, 14336
    w_rows = weight_rows(O.Q4_K, n, k, 7300)
    x = activations(2, k, 7301)
    a = O.quantize_act(O.ACT_Q8_K, x)
    w = dq.Weight.upload(O.Q4_K, w_rows, k)
    ad = dev(a)
    y1 = host(T.gemv(w, O.ACT_Q8_K, ad[:1]))
    y2 = host(T.gemv(w, O.ACT_Q8_K, ad))
    assert np.array_equal(bits(y1[0]), bits(y2[0]))
    rows = np.random.default_rng(7302).choice(n, 256, replace=False)
    want = O.matmul(O.Q4_K, O.ACT_Q8_K, w_rows[rows], a[:1], k)
    assert np.array_equal(bits(y1[0, rows]), bits(want[0]))
    assert np.array_equal(bits(host(T.matmul(w, dev(x[:1])))), bits(y1))
    w.free()
