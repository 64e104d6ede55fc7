"""GPU parity of the K-quant decode GEMV with the per-32 quantization fused into it
(qmm's int8 gemv contract, dq_matmul_act(DQ_ACT_PER32) on Q4_K weights up to 4 rows and
Q6_K up to 2 (from 5 and 3 rows they take the f16 GEMMs, tests/test_gpu_gemm_p32.py and
tests/test_gpu_gemm_q6x.py), and so the default plan's decode): each wave quantizes its
slice of the fp32
rows with the standalone per-32 quantizer's device function, so the codes, and then
every output bit, equal dq_act_quantize followed by dq_gemv on the same rows. Cases:
1 to 4 rows (Q6_K: to 2), super-block counts of 1, 5, 8 and 16 (one Q4_K row of 8 or 16 runs on
56-row workgroups, k_gemv_slab), config 3's full gate shape, a long Q6_K row that the
GEMV splits over K (K = 14336), and rows x_stride > k floats apart; plus the oracle's
per-32 order within the north-star tolerance.

Reference style: dynacore/tests/test_qmm.cpp:178-282 (tier equality).
"""
from __future__ import annotations

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import activations, close, gguf_weights
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


CASES = [(O.Q4_K, 1, 4096, 1000), (O.Q4_K, 1, 2048, 130), (O.Q4_K, 3, 1280, 300), (O.Q4_K, 4, 256, 200),
         (O.Q4_K, 4, 4096, 130), (O.Q6_K, 1, 4096, 1000), (O.Q6_K, 1, 2048, 130), (O.Q6_K, 2, 1280, 300),
         (O.Q6_K, 2, 256, 200), (O.Q6_K, 2, 4096, 130)]


@pytest.mark.parametrize("t,m,k,n", CASES, ids=lambda v: str(v))
def test_fused_per32_equals_quantize_then_gemv(cuda, t, m, k, n):
    import dqtorch as T

    w_rows = gguf_weights(t, n, k, 8800 + m + t, outlier_frac=0.01)
    x = activations(m, k, 8801 + m, outliers=True)
    w = dq.Weight.upload(t, w_rows, k)
    xp = np.zeros((m, k + 24), np.float32)
    xp[:, :k] = x
    xd = torch.from_numpy(xp).cuda()[:, :k]
    bias = torch.from_numpy(np.linspace(-1, 1, n, dtype=np.float32)).cuda()
    fused = host(T.matmul_act(w, O.ACT_PER32, xd, bias=bias))
    two = host(T.gemv(w, O.ACT_PER32, T.quantize(O.ACT_PER32, xd), bias=bias))
    assert np.array_equal(fused.view(np.uint32), two.view(np.uint32))
    want = O.matmul(t, O.ACT_PER32, w_rows, O.quantize_act(O.ACT_PER32, x), k, bias=bias.cpu().numpy())
    ok, worst = close(fused, want)
    assert ok, f"worst error ratio {worst:.3g}"
    w.free()


def test_fused_per32_long_q6k_rows(cuda):
    """Config 3's down projection (Q6_K K=14336 N=4096) at one row: the GEMV splits K over
    workgroups, each quantizing only its own range."""
    import dqtorch as T

    k, n = 14336, 4096
    w_rows = gguf_weights(O.Q6_K, n, k, 8900, outlier_frac=0.01)
    x = activations(1, k, 8901, outliers=False)
    w = dq.Weight.upload(O.Q6_K, w_rows, k)
    xd = torch.from_numpy(x).cuda()
    fused = host(T.matmul_act(w, O.ACT_PER32, xd))
    two = host(T.gemv(w, O.ACT_PER32, T.quantize(O.ACT_PER32, xd)))
    assert np.array_equal(fused.view(np.uint32), two.view(np.uint32))
    w.free()


def test_fused_per32_config3_shape(cuda):
    """Config 3's gate shape (Q4_K K=4096 N=14336) at one row: the default plan's decode
    (256 workgroups of 56 rows) equals the two-launch route on every row."""
    import dqtorch as T

    k, n = 4096, 14336
    w_rows = gguf_weights(O.Q4_K, n, k, 8950, outlier_frac=0.01)
    x = activations(1, k, 8951, outliers=False)
    w = dq.Weight.upload(O.Q4_K, w_rows, k)
    xd = torch.from_numpy(x).cuda()
    fused = host(T.matmul_act(w, O.ACT_PER32, xd))
    two = host(T.gemv(w, O.ACT_PER32, T.quantize(O.ACT_PER32, xd)))
    assert np.array_equal(fused.view(np.uint32), two.view(np.uint32))
    rows = np.random.default_rng(8952).choice(n, 128, replace=False)
    want = O.matmul(O.Q4_K, O.ACT_PER32, w_rows[rows], O.quantize_act(O.ACT_PER32, x), k)
    ok, worst = close(fused[:, rows], want)
    assert ok, f"worst error ratio {worst:.3g}"
    w.free()
