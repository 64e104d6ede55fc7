"""The fp32 expand + GEMM class on the CPU: the oracle's restatement of the x86
weight expansion (dqo_expand_x86, kernels_avx2.cpp:370-466) pinned against the
reference's own outputs (tests/golden/expand_vectors.npz, written by
tests/golden/make_expand_golden.py from oracle/_ref), against the live reference build
where it exists, and against values worked out by hand; and the reference's own
expand + GEMM outputs against the exact product of the expanded operands."""
from __future__ import annotations

import os
import struct

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TYPES = (O.Q8_0, O.Q4_0, O.Q4_K, O.Q6_K)


@pytest.fixture(scope="module")
def ev():
    return np.load(os.path.join(GOLDEN, "expand_vectors.npz"))


@pytest.fixture(scope="module")
def rv():
    return np.load(os.path.join(GOLDEN, "reference_vectors.npz"))


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_expand_matches_reference_golden(ev, rv, t):
    name = O.TYPE_NAMES[t]
    assert np.array_equal(bits(O.expand_x86(t, rv[f"w_{name}"], 512)), bits(ev[f"exp_{name}"]))
    rw = ev[f"rw_{name}"]
    k = ev[f"exp_rw_{name}"].shape[1]
    assert np.array_equal(bits(O.expand_x86(t, rw[:8], k)), bits(ev[f"exp_rw_{name}"]))


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs the reference sources)")
@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_expand_matches_reference_live(t):
    """Random block bytes (any scales and codes; fp16 d kept finite) through both."""
    if not O.ref().ref_has_avx2():
        pytest.skip("no AVX2 on this host")
    k = 1024
    rng = np.random.default_rng(90 + t)
    rows = rng.integers(0, 256, (32, O.row_bytes(t, k)), dtype=np.uint8)
    be = 256 if t in (O.Q4_K, O.Q6_K) else 32
    bb = O.row_bytes(t, be)
    blk = rows.reshape(32, k // be, bb)
    d_at = {O.Q8_0: [0], O.Q4_0: [0], O.Q4_K: [0, 2], O.Q6_K: [208]}[t]
    for off in d_at:  # finite fp16 scales of either sign
        h = O.fp32_to_fp16(rng.uniform(-0.05, 0.05, (32, k // be)).astype(np.float32))
        blk[:, :, off:off + 2] = h.view(np.uint8).reshape(32, k // be, 2)
    assert np.array_equal(bits(O.expand_x86(t, rows, k)), bits(O.ref_expand_x86(t, rows, k)))


def test_expand_known_answers():
    """Hand-built blocks: each value is code * scale (+ the min term), with the
    scales read from the formats' documented positions."""
    # Q4_K: d = 0.5, dmin = 0.25; sub-block 0: sc 3, m 2; sub-block 5: sc 33 (bits
    # 0-3 in byte 9, bits 4-5 in byte 1's top), m 17 (byte 9 high nibble, byte 5 top)
    blk = bytearray(144)
    blk[0:2] = np.float16(0.5).tobytes()
    blk[2:4] = np.float16(0.25).tobytes()
    sc = bytearray(12)
    sc[0], sc[4] = 3, 2
    sc[9] = (33 & 15) | ((17 & 15) << 4)
    sc[1] |= (33 >> 4) << 6
    sc[5] |= (17 >> 4) << 6
    blk[4:16] = sc
    qs = bytearray(128)
    qs[7] = 0x09 | (0x0C << 4)  # value 7 (sub-block 0, low nibble) = 9; value 39 (sub-block 1) = 12
    qs[32 + 10] = 0x0E << 4  # value 64 + 10 = 74 (low nibble) = 0; value 64 + 32 + 10 = 106 (high) = 14
    qs[64 + 5] = 0x07 << 4  # value 128 + 32 + 5 = 165: sub-block 5, code 7
    blk[16:] = qs
    y = O.expand_x86(O.Q4_K, np.frombuffer(bytes(blk), np.uint8), 256)[0]
    assert y[7] == np.float32(0.5 * 3 * 9 - 0.25 * 2)
    assert y[165] == np.float32(0.5 * 33 * 7 - 0.25 * 17)
    assert y[0] == np.float32(-0.25 * 2)  # code 0 leaves the min term alone
    # Q6_K: value 130 = 128 + 2: ql[64 + 2] low nibble | qh[32 + 2] bits 0-1, scale 130 // 16 = 8
    blk = bytearray(210)
    blk[128 + 64 + 0] = 0  # keep the rest zero
    blk[64 + 2] = 0x0B
    blk[128 + 32 + 2] = 0x02
    blk[192 + 8] = struct.pack("b", -3)[0]
    blk[208:210] = np.float16(0.125).tobytes()
    y = O.expand_x86(O.Q6_K, np.frombuffer(bytes(blk), np.uint8), 256)[0]
    assert y[130] == np.float32(0.125 * -3 * ((0x0B | (2 << 4)) - 32))
    # Q4_0: value 20 = high nibble of byte 4, minus 8
    blk = bytearray(18)
    blk[0:2] = np.float16(2.0).tobytes()
    blk[2 + 4] = 0x3 << 4
    y = O.expand_x86(O.Q4_0, np.frombuffer(bytes(blk), np.uint8), 32)[0]
    assert y[20] == np.float32(2.0 * (3 - 8)) and y[4] == np.float32(2.0 * -8)


def _exact(t, rows, x, k):
    w = O.expand_x86(t, rows, k).astype(np.float64)
    xf = np.asarray(x, np.float64)
    return xf @ w.T, np.abs(xf) @ np.abs(w).T


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_reference_expand_gemm_is_within_the_class_bound(ev, rv, t):
    """The reference's own expand + GEMM outputs lie within 1e-6 sum |terms| of the exact
    product of the expanded operands (so the class bound the GPU is held to, 1e-5,
    is not a loose copy of the reference's error)."""
    name = O.TYPE_NAMES[t]
    exact, mag = _exact(t, rv[f"w_{name}"], rv["act_x"], 512)
    assert np.all(np.abs(ev[f"expgemm_{name}"] - exact) <= 1e-6 * mag)
    rw, gx = ev[f"rw_{name}"], ev[f"gx_{name}"]
    exact, mag = _exact(t, rw, gx, gx.shape[1])
    assert np.all(np.abs(ev[f"expgemm_rw_{name}"] - exact) <= 1e-6 * mag)


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs the reference sources)")
def test_cpu_baseline_call_computes_the_decode_step():
    """bench.py's CPU baseline (ref_bench_decode_sx: quantize_act_sx + the sub-scaled row
    kernel on the reference's ThreadPool) writes the decode step's outputs, on 1 and 3
    threads: bit-equal to the same reference kernel called once over all rows (so the
    pool's partition covers every row once), and within the sub-scaled class's fp32
    reordering bound of the oracle."""
    import ctypes as C

    r = O.ref()
    if not r.ref_has_avx2():
        pytest.skip("no AVX2 on this host")
    k, n = 1024, 200
    rng = np.random.default_rng(77)
    rows = rng.integers(0, 256, (n, k // 256, 144), dtype=np.uint8)
    rows[:, :, 0:4] = rng.uniform(0.002, 0.02, (n, k // 256, 2)).astype(np.float16).view(np.uint8).reshape(n, -1, 4)
    rows = np.ascontiguousarray(rows.reshape(n, -1))
    x = O.normal(78, k)
    a = O.ref_quantize("sx", x)
    whole = np.empty(n, np.float32)
    assert r.ref_dot_rows_n(3, O.Q4_K, rows.ctypes.data, rows.shape[1], 0, n, a.ctypes.data, a.size, 1, k,
                            whole.ctypes.data, n, None) == 0
    oracle = O.matmul(O.Q4_K, O.ACT_SX, rows, a.reshape(1, -1), k)[0]
    ptrs = (C.c_void_p * 1)(rows.ctypes.data)
    for threads in (1, 3):
        y = np.full(n, np.nan, np.float32)
        assert r.ref_bench_decode_sx(O.Q4_K, ptrs, 1, rows.shape[1], n, x.ctypes.data, 1, k, y.ctypes.data, threads,
                                     32, 1) > 0
        assert np.array_equal(y.view(np.uint32), whole.view(np.uint32))
        assert np.max(np.abs(y - oracle)) <= 1e-5 * np.abs(oracle).max()
    assert r.ref_llc_bytes() >= 0
