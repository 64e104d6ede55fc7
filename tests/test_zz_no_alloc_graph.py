"""dq_matmul_noalloc under HIP graph capture, the callers its declaration names.

A fresh child process captures dq_matmul_noalloc into a torch.cuda.graph before any
other call of it, so the capture holds the first call on the device: the one-time
lookup of the static array's device address and the launches' attribute calls happen
while the stream is capturing. Each route that uses the array (the f16 Q4_K GEMM, the
per-32 block GEMM, the skinny MFMA passes, the split-K decode GEMV, the split skinny
launch with its t-terms and chain launch) is captured as its
first call for that weight and shape; every replay, with eager work on the same
buffers between replays, equals eager dq_matmul bit for bit."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import sys
sys.path.insert(0, ROOT)
sys.path.insert(0, ROOT + "/tests")
import torch
import dynalm_amd as dq
from dqtest import activations, gguf_weights

# (name, dtype, n, k, m): one route of dq_matmul that uses the array each
CASES = [("q4k-f16-gemm", dq.Q4_K, 14336, 4096, 512), ("q4_0-b32-gemm", dq.Q4_0, 2048, 4096, 64),
         ("q6k-skinny", dq.Q6_K, 1536, 1536, 40), ("q8_0-splitk", dq.Q8_0, 4096, 14336, 3),
         ("q6k-skinny-split", dq.Q6_K, 1536, 8960, 16)]
for name, t, n, k, m in CASES:
    print("case", name, flush=True)
    w = dq.Weight.upload(t, gguf_weights(t, n, k, 700 + t), k)
    x = torch.from_numpy(activations(m, k, 701 + t)).cuda()
    y_g = torch.full((m, n), 5.0, device="cuda")
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        rc = dq.lib().dq_matmul_noalloc(w.handle, x.data_ptr(), m, k, y_g.data_ptr(), n, None, side.cuda_stream)
    assert rc == 0, (name, rc, dq.lib().dq_last_error().decode())
    y_ref = torch.empty((m, n), device="cuda")
    dq.matmul(w, x, m, k, y_ref, n, None, torch.cuda.current_stream().cuda_stream)
    for rep in range(3):
        y_g.fill_(float(rep))          # eager work on the output between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_g.view(torch.int32), y_ref.view(torch.int32)), (name, rep)
    del g
    w.free()
    print("ok", name, flush=True)
"""


def test_noalloc_graph_capture_first_call(cuda):
    env = dict(os.environ)
    res = subprocess.run([sys.executable, "-c", "ROOT = " + repr(ROOT) + "\n" + CHILD], capture_output=True, text=True,
                         timeout=300, env=env)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-3000:]
    for name in ("q4k-f16-gemm", "q4_0-b32-gemm", "q6k-skinny", "q8_0-splitk", "q6k-skinny-split"):
        assert f"ok {name}" in res.stdout, out[-3000:]
