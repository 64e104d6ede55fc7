"""dq_matmul_noalloc: dq_matmul with its temporaries in the library's static device
array. Through the C ABI, every route dq_matmul takes gives the same bits on two
calls in a row, the second with a smaller input (the array keeps the first call's
contents); a call needing more than the array holds fails before launching."""
from __future__ import annotations

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import activations, gguf_weights
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _both(w: dq.Weight, x: np.ndarray):
    """(dq_matmul, dq_matmul_noalloc) outputs for fp32 rows x."""
    m = x.shape[0]
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    y_ref = torch.full((m, w.n), 7.0, device="cuda")
    y_na = torch.full((m, w.n), 9.0, device="cuda")
    dq.matmul(w, xd, m, xd.stride(0), y_ref, y_ref.stride(0), None, _stream())
    rc = dq.lib().dq_matmul_noalloc(w.handle, xd.data_ptr(), m, xd.stride(0), y_na.data_ptr(), y_na.stride(0), None,
                                    _stream())
    assert rc == 0, dq.lib().dq_last_error().decode()
    torch.cuda.synchronize()
    return y_ref.cpu().numpy(), y_na.cpu().numpy()


# (name, dtype, n, k, first m, second m): each route of dq_matmul that uses scratch
CASES = [
    ("q4k-gemm", O.Q4_K, 14336, 4096, 512, 64),      # quantize + MFMA GEMM (2.4 MB of Q8_K rows), then smaller
    ("q8_0-splitk", O.Q8_0, 4096, 14336, 3, 1),      # fused GEMV with split-K row sums in the array
    ("q6k-skinny", O.Q6_K, 1536, 1536, 40, 16),       # quantize + skinny passes, then the fused skinny launch
    ("q4_0-b32gemm", O.Q4_0, 2048, 4096, 64, 2),      # per-32 quantize + block GEMM, then the fused GEMV
    ("q6k-down-gemm", O.Q6_K, 4096, 14336, 200, 17),  # Q6_K large GEMM at K = 14336
    ("q6k-down-split", O.Q6_K, 1536, 8960, 16, 7),    # quantize + split skinny (t-terms in the array) + chains
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_noalloc_equals_matmul_twice(cuda, case):
    _, t, n, k, m1, m2 = case
    w = dq.Weight.upload(t, gguf_weights(t, n, k, 900 + t), k)
    for i, m in enumerate((m1, m2)):
        x = activations(m, k, 901 + i)
        ref, na = _both(w, x)
        assert np.array_equal(ref.view(np.uint32), na.view(np.uint32)), f"call {i + 1} (m={m})"


def test_noalloc_rejects_oversize(cuda):
    """More rows than the array's scratch holds: DQ_RESOURCE_EXHAUSTED, y untouched."""
    k, n = 4096, 256
    w = dq.Weight.upload(O.Q4_K, gguf_weights(O.Q4_K, n, k, 950), k)
    m = dq.NOALLOC_SCRATCH_BYTES // dq.act_row_bytes(dq.ACT_Q8_K, k) + 1
    x = torch.zeros((m, k), device="cuda")
    y = torch.full((m, n), 3.0, device="cuda")
    rc = dq.lib().dq_matmul_noalloc(w.handle, x.data_ptr(), m, k, y.data_ptr(), n, None, _stream())
    assert rc == 5, rc  # DQ_RESOURCE_EXHAUSTED
    assert b"DQ_NOALLOC_SCRATCH_BYTES" in dq.lib().dq_last_error()
    torch.cuda.synchronize()
    assert bool(torch.all(y == 3.0))
    # one row fewer fits
    ref, na = _both(w, activations(m - 1, k, 951, outliers=False))
    assert np.array_equal(ref.view(np.uint32), na.view(np.uint32))
