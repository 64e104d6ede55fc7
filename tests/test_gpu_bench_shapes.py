"""GPU parity at the exact shapes bench.py times, and on the launch variants only those
shapes select.

- The large GEMM kernels over many super-blocks: Q4_K K=4096 N=14336 at M=512 and
  M=2048 (the f16 128 x 256 kernel: one round of 224 workgroups, and 3.5 rounds),
  Q6_K over 4 and 56 super-blocks (the 256 x 128 tile). Every output bit-identical to the GEMV on the same Q8_K rows,
  sampled columns bit-identical to the oracle.
- The per-32 GEMM (Q8_0 4096 x 4096, Q4_0 K=4096 N=14336) at M=512.
- The 4-wave gated skinny launch at config 5's gate/up shape (Q4_K 8960 x 1536, M=16).
- dq_matmul's fused decode path at K = 14336 (split-K for the per-32 formats, the
  early-activation GEMV for the K-quants), equal to quantize + dq_gemv bit for bit.
- Row-range calls whose row-group count differs from the full call's: the K partition
  of a row depends only on the weight, so the bits equal the full call's.

Reference style: dynacore/tests/test_qmm.cpp:178-282 (odd M, split ranges, tier equality).
"""
from __future__ import annotations

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import activations, close, gguf_weights, weight_rows
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


@pytest.mark.parametrize("m", [512, 2048])
def test_gemm_q4k_bench_shape(cuda, m):
    """Config 4 (K=4096, N=14336) at the bench's M: k_gemm_q4k_h16 over 16 super-blocks
    (through its ring of two LDS operand buffers), one round of 224 workgroups at M=512
    and 3.5 rounds at M=2048. dq_gemm == dq_gemv bit for bit on every output; 128 sampled columns ==
    the oracle bit for bit; dq_matmul (quantize + GEMM) == quantize then dq_gemm."""
    import dqtorch as T

    k, n = 4096, 14336
    w_rows = weight_rows(O.Q4_K, n, k, 4000 + m, edge=True)
    x = activations(m, k, 4001 + m)
    w = dq.Weight.upload(O.Q4_K, w_rows, k)
    xd = dev(x)
    ad = T.quantize(O.ACT_Q8_K, xd)
    a = host(ad)
    assert np.array_equal(a, O.quantize_act(O.ACT_Q8_K, x))
    yg = host(T.gemm(w, O.ACT_Q8_K, ad))
    yv = host(T.gemv(w, O.ACT_Q8_K, ad))
    assert np.array_equal(bits(yg), bits(yv)), "GEMM differs from the GEMV"
    cols = np.random.default_rng(m).choice(n, 128, replace=False)
    want = O.matmul(O.Q4_K, O.ACT_Q8_K, w_rows[cols], a, k)
    assert np.array_equal(bits(yg[:, cols]), bits(want)), "GEMM differs from the oracle"
    ym = host(T.matmul(w, xd))
    assert np.array_equal(bits(ym), bits(yg)), "dq_matmul differs from quantize + dq_gemm"


@pytest.mark.parametrize("t,n,k", [(O.Q8_0, 4096, 4096), (O.Q4_0, 14336, 4096)], ids=["q8_0", "q4_0"])
def test_gemm_b32_bench_shape(cuda, t, n, k):
    """The per-32 GEMM at the shapes the bench times (M=512): k_gemm_b32 over 128 blocks, 32
    stages through its two LDS stage buffers, 512 / 1,792 workgroups (one round / 2.3 rounds
    of three per CU). 128 sampled columns == the oracle bit for bit; dq_matmul (quantize +
    GEMM) == quantize then dq_gemm on every output."""
    import dqtorch as T

    m = 512
    w_rows = weight_rows(t, n, k, 4500 + t, edge=True)
    x = activations(m, k, 4501)
    w = dq.Weight.upload(t, w_rows, k)
    xd = dev(x)
    ad = T.quantize(O.ACT_PER32, xd)
    a = host(ad)
    assert np.array_equal(a, O.quantize_act(O.ACT_PER32, x))
    yg = host(T.gemm(w, O.ACT_PER32, ad))
    cols = np.unique(np.concatenate([np.random.default_rng(t).choice(n, 128, replace=False), [0, n - 1]]))
    want = O.matmul(t, O.ACT_PER32, w_rows[cols], a, k)
    assert np.array_equal(bits(yg[:, cols]), bits(want)), "GEMM differs from the oracle"
    ym = host(T.matmul(w, xd))
    assert np.array_equal(bits(ym), bits(yg)), "dq_matmul differs from quantize + dq_gemm"


@pytest.mark.parametrize("m,n,k", [(512, 14336, 1024), (512, 4096, 14336)])
def test_gemm_q6k_many_superblocks(cuda, m, n, k):
    """The Q6_K large GEMM over several super-blocks: <4, 2, 4> at N=14336 (4 super-blocks)
    and <2, 2, 2> at the FFN-down shape the bench times (K=14336, N=4096: 56 super-blocks).
    Bit-identical to the GEMV on every output and to the oracle on sampled columns."""
    import dqtorch as T

    w_rows = weight_rows(O.Q6_K, n, k, 4100 + k, edge=True)
    x = activations(m, k, 4101 + k)
    w = dq.Weight.upload(O.Q6_K, w_rows, k)
    ad = T.quantize(O.ACT_Q8_K, dev(x))
    a = host(ad)
    yg = host(T.gemm(w, O.ACT_Q8_K, ad))
    yv = host(T.gemv(w, O.ACT_Q8_K, ad))
    assert np.array_equal(bits(yg), bits(yv)), "GEMM differs from the GEMV"
    cols = np.concatenate([np.random.default_rng(k).choice(n, 96, replace=False), [0, n - 1]])
    want = O.matmul(O.Q6_K, O.ACT_Q8_K, w_rows[cols], a, k)
    assert np.array_equal(bits(yg[:, cols]), bits(want)), "GEMM differs from the oracle"


def test_gated_skinny_config5_shape(cuda):
    """Config 5's gate/up pair (Q4_K 8960 x 1536, M=16) through dq_matmul_gated: 560 tiles of 6
    super-blocks (12 counting gate and up) on 256 CUs select the 4-wave gated skinny launch
    after one quantize launch. Every output against the oracle's act(g) * u (SiLU: bit-exact),
    and bit-identical to act_mul over two dq_matmul calls."""
    import dqtorch as T

    n, k, m = 8960, 1536, 16
    rg = gguf_weights(O.Q4_K, n, k, 4200)
    ru = gguf_weights(O.Q4_K, n, k, 4201)
    wg, wu = dq.Weight.upload(O.Q4_K, rg, k), dq.Weight.upload(O.Q4_K, ru, k)
    x = activations(m, k, 4202, outliers=False)
    xd = dev(x)
    out = host(T.matmul_gated(O.SILU, xd, wg, wu))
    comp = host(T.act_mul(O.SILU, T.matmul(wg, xd), T.matmul(wu, xd)))
    assert np.array_equal(bits(out), bits(comp)), "fused differs from act_mul(matmul, matmul)"
    a = O.quantize_act(O.ACT_Q8_K, x)
    g = O.matmul(O.Q4_K, O.ACT_Q8_K, rg, a, k)
    u = O.matmul(O.Q4_K, O.ACT_Q8_K, ru, a, k)
    want = (O.activation(O.SILU, g) * u).astype(np.float32)
    assert np.array_equal(bits(out), bits(want)), "gated output differs from the oracle"


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_0, O.Q4_K, O.Q6_K], ids=lambda t: O.TYPE_NAMES[t])
@pytest.mark.parametrize("n", [256, 4096])
@pytest.mark.parametrize("m", [1, 3])
def test_fused_decode_long_rows(cuda, t, n, m):
    """dq_matmul's fused decode at K = 14336 (the FFN-down length): the per-32 formats split K
    over workgroups (kFuse with kSplit: each workgroup quantizes its K-range), the K-quants at
    M = 1 run the early-activation GEMV (3-4 super-blocks per wave). Bit-identical to the
    standalone quantizer followed by dq_gemv; sampled rows against the oracle (bit-exact for
    Q8_K, within the fp32 bar for per-32)."""
    import dqtorch as T

    k = 14336
    w_rows = gguf_weights(t, n, k, 4300 + t + n)
    x = activations(m, k, 4301 + m)
    w = dq.Weight.upload(t, w_rows, k)
    fmt = dq.act_format_for(t)
    xd = dev(x)
    fused = host(T.matmul(w, xd))
    two = host(T.gemv(w, fmt, T.quantize(fmt, xd)))
    assert np.array_equal(bits(fused), bits(two)), "fused differs from quantize + gemv"
    rows = np.random.default_rng(n + m).choice(n, 48, replace=False)
    want = O.matmul(t, fmt, w_rows[rows], O.quantize_act(fmt, x), k)
    if fmt == O.ACT_Q8_K:
        assert np.array_equal(bits(fused[:, rows]), bits(want))
    else:
        ok, worst = close(fused[:, rows], want)
        assert ok, f"worst error ratio {worst:.3g}"


@pytest.mark.parametrize("t,fmt,k", [(O.Q8_0, O.ACT_PER32, 14336), (O.Q4_0, O.ACT_PER32, 14336),
                                     (O.Q6_K, O.ACT_Q16, 14336), (O.Q4_K, O.ACT_F32, 4096),
                                     (O.Q6_K, O.ACT_PER32, 4096)],
                         ids=["q8_0-per32", "q4_0-per32", "q6_K-q16", "q4_K-f32", "q6_K-per32"])
def test_row_range_matches_full_call(cuda, t, fmt, k):
    """qmm.h:35-36: the caller partitions [n0, n1) and a row's result does not depend on the
    partition. N = 4096 is 64 row groups (the full call splits K); the halves and a ragged
    range have fewer groups, yet each row's bits equal the full call's."""
    import dqtorch as T

    n, m = 4096, 3
    w_rows = gguf_weights(t, n, k, 4400 + t + k)
    x = activations(m, k, 4401)
    w = dq.Weight.upload(t, w_rows, k)
    xd = dev(x)
    acts = T.quantize(fmt, xd)  # DQ_ACT_F32: the rows copied densely
    full = host(T.gemv(w, fmt, acts))
    parts = torch.full((m, n), 123.0, device="cuda")
    for n0, n1 in [(0, 2048), (2048, 4096)]:
        T.gemv(w, fmt, acts, n0=n0, n1=n1, out=parts)
    got = host(parts)
    assert np.array_equal(bits(got), bits(full)), "halves differ from the full call"
    ragged = torch.full((m, n), 123.0, device="cuda")
    T.gemv(w, fmt, acts, n0=70, n1=1000, out=ragged)
    r = host(ragged)
    assert np.array_equal(bits(r[:, 70:1000]), bits(full[:, 70:1000]))
    assert np.all(r[:, :70] == 123.0) and np.all(r[:, 1000:] == 123.0)
