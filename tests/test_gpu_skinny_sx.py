"""GPU parity of the skinny MFMA GEMV on sub-scaled activations (DQ_ACT_SX, dynacore's
default contract for K-quant decode rows, kernels_avx2.cpp:1077-1216): Q4_K / Q6_K x
ActSuperQ8 for 2..16 rows per pass (dq_skinny.hip, tterms on ActSBX).

Each K-step of the kernel spans two 32-value sub-blocks with their own activation
multipliers m_b, so every chain runs once per half step and the products m_b S_b go
into a 64-bit S. dq_gemv takes this kernel where it was measured faster than the VALU
GEMV (skinny_sx_pays: one round of 16-row tiles, Q6_K below the 64-row-tile launches,
or 8 rows and more), else the VALU GEMV. The cases cover each launch shape of the
kernel (16-row tiles with 8 waves, 4-wave workgroups for many tiles, 64-row tiles for
very many, the 2-deep weight ring for long rows), the VALU route on a many-tile launch,
passes of 16 rows (m = 17 ends on one row, which the M = 1 GEMV takes), and the largest
products: Q6_K scales of -128 on codes 0 (q - 32 = -32) against rows whose sub-block
multipliers are all 128, the bound each half step's int32 product is sized for. Every
output is bit-identical to the oracle's order for this contract.
"""
from __future__ import annotations

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import activations, gguf_weights
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


def _check(t: int, n: int, k: int, m: int, seed: int, sample: int | None = None) -> None:
    import dqtorch as T

    rows = gguf_weights(t, n, k, seed, outlier_frac=0.01)
    x = activations(m, k, seed + 1)
    a = O.quantize_act(O.ACT_SX, x)
    w = dq.Weight.upload(t, rows, k)
    y = host(T.gemv(w, O.ACT_SX, dev(a)))
    cols = np.arange(n) if sample is None else np.unique(np.concatenate(
        [np.random.default_rng(seed).choice(n, sample, replace=False), [0, n - 1]]))
    want = O.matmul(t, O.ACT_SX, rows[cols], a, k)
    assert np.array_equal(bits(y[:, cols]), bits(want))
    # dq_matmul_act quantizes on the GPU and runs the same kernel
    ya = host(T.matmul_act(w, O.ACT_SX, dev(x)))
    assert np.array_equal(bits(ya), bits(y))


TYPES = [O.Q4_K, O.Q6_K]
TID = [O.TYPE_NAMES[t] for t in TYPES]


@pytest.mark.parametrize("t", TYPES, ids=TID)
@pytest.mark.parametrize("m", [2, 4, 16])
def test_sx_skinny_8_wave_tiles(cuda, t, m):
    """13 tiles of 16 rows, 5 super-blocks: 8-wave workgroups, one pass."""
    _check(t, 200, 1280, m, 7000 + m + t)


@pytest.mark.parametrize("t", TYPES, ids=TID)
@pytest.mark.parametrize("m", [3, 8])
def test_sx_skinny_4_wave_many_tiles(cuda, t, m):
    """Config 5's gate shape (8960 x 1536): 560 tiles, more than the CUs, 4-wave workgroups
    (Q4_K at 3 rows: the VALU GEMV route)."""
    _check(t, 8960, 1536, m, 7100 + m + t, sample=512)


@pytest.mark.parametrize("t", TYPES, ids=TID)
@pytest.mark.parametrize("m", [3, 8])
def test_sx_skinny_64_row_tiles(cuda, t, m):
    """65,536 rows of one super-block: 4,096 16-row tiles, so 64-row tiles (CT = 4) at 8 rows
    (3 rows: the VALU GEMV route)."""
    _check(t, 65536, 256, m, 7200 + t + m, sample=512)


@pytest.mark.parametrize("t", TYPES, ids=TID)
@pytest.mark.parametrize("m", [4, 16])
def test_sx_skinny_long_rows_ring(cuda, t, m):
    """The FFN down projection's shape (1536 x 8960): 96 tiles of 35 super-blocks, one round
    of workgroups with the 2-deep weight ring."""
    _check(t, 1536, 8960, m, 7300 + m + t, sample=384)


@pytest.mark.parametrize("m", [17, 40])
def test_sx_skinny_passes(cuda, m):
    """More rows than one pass: 16-row passes (m = 17: the last row on the M = 1 GEMV)."""
    _check(O.Q4_K, 200, 1024, m, 7400 + m)


def test_sx_skinny_q6k_largest_products(cuda):
    """Q6_K scales -128 and codes 0 (q - 32 = -32) against constant rows (every m_b = 128,
    codes +-127): each half step's |64 H + L| m_b = 32 * 128 * 32 * 127 * 128, the int32
    bound of the kernel's products, and S far beyond 2^31 in the 64-bit sum."""
    import dqtorch as T

    k, n = 512, 64
    blk = np.zeros(210, np.uint8)
    blk[192:208] = 0x80                                       # int8 scales -128
    blk[208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    rows = np.tile(np.tile(blk, k // 256)[None, :], (n, 1))
    rows[1::2, 0:128] = 0xFF                                  # odd rows: low nibbles 15
    x = np.full((3, k), 3.0, np.float32)
    x[1] *= -1.0
    x[2, ::2] *= -1.0
    a = O.quantize_act(O.ACT_SX, x)
    w = dq.Weight.upload(O.Q6_K, rows, k)
    y = host(T.gemv(w, O.ACT_SX, dev(a)))
    want = O.matmul(O.Q6_K, O.ACT_SX, rows, a, k)
    assert np.array_equal(bits(y), bits(want))
    assert abs(float(want[0, 0])) > 0
