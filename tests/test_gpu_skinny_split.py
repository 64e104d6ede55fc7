"""GPU parity of the split skinny launch (k_skinny_split + k_skinny_chain,
dq_skinny.hip): Q6_K weights x Q8_K activations at 2..16 rows with long rows (32 to
64 super-blocks) on at most half as many 16-row tiles as CUs, e.g. config 5's FFN
down projection (Q6_K 1536 x 8960: 96 tiles). Workgroups of one 64-row group x 4
super-blocks write the t-terms to a buffer (the caller's region or the stream's
workspace) and a second launch runs the in-order chains. Q4_K at the same shapes,
and Q6_K on 256 tiles, take k_skinny: the same checks hold them to the same bar.

Bar: bit-identical to the oracle (the Q8_K pairs' integer S, Mn and canonical fp32
steps), as every other route of these pairs. Cases: 32, 35, 39, 56 and 64
super-blocks, 2 / 7 / 9 / 16 activation rows, weight row counts that end inside a
16-row tile, row ranges that start in a later 64-row group, a bias, the reference's
edge blocks, both entry routes (dq_gemv on Q8_K rows, dq_matmul on fp32 rows), and
a grouped launch of two jobs (dq_matmul_many, which stays unsplit).

Reference style: dynacore/tests/test_qmm.cpp:178-282 (odd shapes, split ranges).
"""
from __future__ import annotations

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import activations, gguf_weights, weight_rows
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TYPES = [O.Q4_K, O.Q6_K]


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
@pytest.mark.parametrize("m,n,k", [(16, 1536, 8960), (7, 1000, 8192), (2, 40, 9984), (16, 203, 9984), (9, 1024, 16384),
                                   (9, 4096, 14336)])
def test_split_bit_exact(cuda, t, m, n, k):
    import dqtorch as T

    seed = 8000 + m + n + t
    w_rows = weight_rows(t, n, k, seed, edge=True)
    x = activations(m, k, seed + 1)
    a = O.quantize_act(O.ACT_Q8_K, x)
    bias = O.normal(seed + 2, n)
    w = dq.Weight.upload(t, w_rows, k)
    want = O.matmul(t, O.ACT_Q8_K, w_rows, a, k, bias=bias)
    y = host(T.gemv(w, O.ACT_Q8_K, dev(a), bias=dev(bias)))
    assert np.array_equal(bits(y), bits(want))
    want_nb = O.matmul(t, O.ACT_Q8_K, w_rows, a, k)
    for n0, n1 in ((9, n - 5), (min(70, n - 2), n - 1)):
        out = torch.full((m, n), 777.0, device="cuda")
        y2 = host(T.gemv(w, O.ACT_Q8_K, dev(a), n0=n0, n1=n1, out=out))
        assert np.all(y2[:, :n0] == 777.0) and np.all(y2[:, n1:] == 777.0)
        assert np.array_equal(bits(y2[:, n0:n1]), bits(want_nb[:, n0:n1]))
    y3 = host(T.matmul(w, dev(x), bias=dev(bias)))  # fp32 rows: quantize launch, then the split launch
    assert np.array_equal(bits(y3), bits(want))
    w.free()


def test_split_grouped_jobs_unsplit(cuda):
    """dq_matmul_many with a Q6_K and a Q4_K job of the same row length (35
    super-blocks) on different fp32 inputs: one quantize launch per input and one
    grouped k_skinny launch (groups of several jobs are not split); each output
    bit-identical to the oracle."""
    k = 8960
    jobs, want = [], []
    for i, (t, n) in enumerate([(O.Q6_K, 1536), (O.Q4_K, 512)]):
        w_rows = gguf_weights(t, n, k, 8100 + i, outlier_frac=0.01)
        x = activations(16, k, 8110 + i, outliers=False)
        w = dq.Weight.upload(t, w_rows, k)
        y = torch.empty((16, n), device="cuda")
        jobs.append((w, dev(x), 16, k, y, n, None))
        want.append(O.matmul(t, O.ACT_Q8_K, w_rows, O.quantize_act(O.ACT_Q8_K, x), k))
    dq.matmul_many(jobs, torch.cuda.current_stream().cuda_stream)
    for job, wv in zip(jobs, want):
        assert np.array_equal(bits(host(job[4])), bits(wv))
        job[0].free()
