"""The CPU oracle, pinned (CPU only).

Each oracle function is checked against something it does not share code with:
the reference's own outputs (committed golden vectors from its compiled kernels,
and the live build in oracle/_ref where present), numpy's IEEE conversions,
independent bit-field decoders, brute-force integer sums and the reference
tests' double-precision bounds. A planted mistake in the oracle (dropped term,
wrong sign / index / rounding) fails at least one of these.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from dqtest import BLOCK, TYPES, activations, gguf_weights, weight_rows
from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_vectors.npz")
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref (reference build) not present")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ------------------------------------------------------------------ fp16


def test_fp16_to_fp32_exhaustive_vs_numpy():
    h = np.arange(65536, dtype=np.uint16)
    mine = O.fp16_to_fp32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(mine), nan)
    assert np.array_equal(mine[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp32_to_fp16_vs_numpy():
    rng = np.random.default_rng(3)
    halves = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    halves = halves[np.isfinite(halves)].astype(np.float64)
    f = np.concatenate([
        rng.integers(0, 2**32, 400000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        halves.astype(np.float32),
        (halves * (1 + 2.0**-11)).astype(np.float32),   # exact midpoints (ties to even)
        (halves * (1 + 2.0**-12)).astype(np.float32),
        np.array([65504, 65519.996, 65520, 1e9, 2.0**-25, 2.0**-24 * 1.5, 2.0**-26, -0.0], np.float32),
    ])
    f = f[np.isfinite(f)]
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.fp32_to_fp16(f), ref)
    nan = np.array([np.nan, -np.nan], np.float32)
    assert list(O.fp32_to_fp16(nan)) == [0x7E00, 0xFE00]


def test_fp16_golden(gold):
    h = np.arange(65536, dtype=np.uint16)
    mine, ref = O.fp16_to_fp32(h), gold["fp16_f"]
    assert np.array_equal(np.isnan(mine), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(mine[ok].view(np.uint32), ref[ok].view(np.uint32))
    assert np.array_equal(O.fp32_to_fp16(gold["f2h_f"]), gold["f2h_h"])


# ---------------------------------------------------- Q4_K scale unpacking


def _scale_min_bitfields(s: bytes, j: int) -> tuple[int, int]:
    """Independent statement of the 12-byte layout as bit fields of a 96-bit integer:
    scales 0-3 = bits 0-5 of bytes 0-3, mins 0-3 = bits 0-5 of bytes 4-7; scales 4-7 =
    low nibble of bytes 8-11 + (bits 6-7 of bytes 0-3) << 4; mins 4-7 = high nibble
    of bytes 8-11 + (bits 6-7 of bytes 4-7) << 4."""
    v = int.from_bytes(s, "little")
    byte = lambda i: (v >> (8 * i)) & 0xFF  # noqa: E731
    if j < 4:
        return byte(j) & 0x3F, byte(4 + j) & 0x3F
    i = j - 4
    return (byte(8 + i) & 0xF) | ((byte(i) >> 6) << 4), (byte(8 + i) >> 4) | ((byte(4 + i) >> 6) << 4)


def test_scale_min_k4_brute_force():
    import ctypes as C

    lib = O.lib()
    sc, mn = C.c_uint8(), C.c_uint8()
    rng = np.random.default_rng(5)
    for j in range(8):
        # every value of each byte that j reads, other bytes random
        for v in range(256):
            for pos in {j % 4, 4 + j % 4, 8 + j % 4}:
                s = bytearray(rng.integers(0, 256, 12, dtype=np.uint8).tobytes())
                s[pos] = v
                buf = (C.c_uint8 * 12).from_buffer_copy(bytes(s))
                lib.dqo_scale_min_k4(j, C.addressof(buf), C.addressof(sc), C.addressof(mn))
                assert (sc.value, mn.value) == _scale_min_bitfields(bytes(s), j)


# ------------------------------------------------------------- quantizers


@pytest.mark.parametrize("kind,fmt", [("q8_0", O.ACT_Q8_0), ("per32", O.ACT_PER32), ("sx", O.ACT_SX)])
def test_act_quantizers_golden(gold, kind, fmt):
    assert np.array_equal(O.quantize_act(fmt, gold["act_x"]), gold[f"act_{kind}"])


def test_act_q16_golden(gold):
    """int16 activations bit-equal to the reference's AVX2 quantize_act16 on the
    seeded rows and the edge row (ties, zero block, +-inf, full scale, tiny values)."""
    assert np.array_equal(O.quantize_act(O.ACT_Q16, gold["q16_x"]), gold["act_q16"])


def test_q16_invariants_and_split(gold):
    """test_int_kernels.cpp:166-178: |x - d q| <= d (0.5 + 3e-7 |q|), sum == sum(q), the
    amax element at +-32767; and the reference's split_act16 bytes are q = 256 hi + lo
    with hi = q >> 8 (signed) and lo = q & 255, the decomposition the GPU kernels use."""
    x = activations(6, 1024, 12)
    a = O.quantize_act(O.ACT_Q16, x).reshape(6, -1, 72)
    d = a[:, :, 0:4].copy().view(np.float32)[..., 0].astype(np.float64)
    s = a[:, :, 4:8].copy().view(np.int32)[..., 0]
    q = a[:, :, 8:].copy().view(np.int16).astype(np.int64)
    xb = x.reshape(6, -1, 32).astype(np.float64)
    assert np.all(np.abs(xb - d[..., None] * q) <= d[..., None] * (0.5 + 3e-7 * np.abs(q)) + 1e-12)
    assert np.array_equal(q.sum(-1), s)
    amax_at = np.abs(xb).argmax(-1)
    qa = np.take_along_axis(q, amax_at[..., None], -1)[..., 0]
    assert np.all(np.abs(qa[d > 0]) == 32767)
    sp = gold["split_q16"].reshape(-1, 72)
    g = gold["act_q16"].reshape(-1, 72)
    assert np.array_equal(sp[:, :8], g[:, :8])
    q = g[:, 8:].copy().view(np.int16).astype(np.int64)
    hi = sp[:, 8:40].view(np.int8).astype(np.int64)
    lo = sp[:, 40:72].astype(np.int64)
    assert np.array_equal(256 * hi + lo, q)
    assert np.array_equal(hi, q >> 8) and np.array_equal(lo, q & 255)


def test_q16_edge_codes():
    """Ties round half to even at d = 1; +-inf give d = inf, id = 0 and the INT32_MIN
    code of cvtps_epi32 (saturated to -32768; two of them wrap the sum to 0)."""
    x = np.zeros((1, 64), np.float32)
    x[0, 0] = 32767.0
    x[0, 1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 32766.5, -32766.5]
    x[0, 32 + 3] = np.inf
    a = O.quantize_act(O.ACT_Q16, x)[0]
    q = a[8:72].copy().view(np.int16)
    assert a[:4].view(np.float32)[0] == 1.0
    assert list(q[1:9]) == [0, 2, 2, 0, -2, -2, 32766, -32766]
    b = a[72:]
    assert b[:4].view(np.float32)[0] == np.inf
    assert b[4:8].view(np.int32)[0] == -2**31
    qb = b[8:].copy().view(np.int16)
    assert qb[3] == -32768 and not np.any(np.delete(qb, 3))


def test_act_q8_K_golden(gold):
    x = gold["act_x"]
    mine = O.quantize_act(O.ACT_Q8_K, x).reshape(x.shape[0], -1, 292)
    sb = gold["act_sb"].reshape(x.shape[0], -1, 40)  # ActBlockQ8 with one d per 8 blocks
    assert np.array_equal(mine[:, :, 4:260].reshape(x.shape[0], -1), sb[:, :, 8:].reshape(x.shape[0], -1))
    assert np.array_equal(mine[:, :, 0:4], sb[:, ::8, 0:4])
    codes = mine[:, :, 4:260].view(np.int8).astype(np.int32).reshape(x.shape[0], -1, 16, 16)
    bsums = mine[:, :, 260:292].copy().view(np.int16).reshape(x.shape[0], -1, 16)
    assert np.array_equal(codes.sum(-1), bsums)


def test_per32_invariants():
    """test_int_kernels.cpp:119-128: |x - d q| <= d (0.5 + 3e-7 |q|), sum == sum(q), and
    the amax element maps to +-127."""
    x = activations(6, 1024, 11)
    a = O.quantize_act(O.ACT_PER32, x).reshape(6, -1, 40)
    d = a[:, :, 0:4].copy().view(np.float32)[..., 0].astype(np.float64)
    s = a[:, :, 4:8].copy().view(np.int32)[..., 0]
    q = a[:, :, 8:].view(np.int8).astype(np.int64)
    xb = x.reshape(6, -1, 32).astype(np.float64)
    assert np.all(np.abs(xb - d[..., None] * q) <= d[..., None] * (0.5 + 3e-7 * np.abs(q)) + 1e-12)
    assert np.array_equal(q.sum(-1), s)
    amax_at = np.abs(xb).argmax(-1)
    qa = np.take_along_axis(q, amax_at[..., None], -1)[..., 0]
    nz = d > 0
    assert np.all(np.abs(qa[nz]) == 127)
    assert np.all(q[~nz] == 0)


def test_rounding_ties_separate_the_two_rules():
    """amax = 127 gives d = 1 and id = 1, so x = k + 0.5 is an exact tie: per-32
    rounds half to even, GGUF Q8_0 rounds half away from zero."""
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 127.0
    x[0, 1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, -3.5]
    per32 = O.quantize_act(O.ACT_PER32, x)[0, 8:].view(np.int8)
    q80 = O.quantize_act(O.ACT_Q8_0, x)[0, 2:].view(np.int8)
    assert list(per32[1:9]) == [0, 2, 2, 0, -2, -2, 4, -4]
    assert list(q80[1:9]) == [1, 2, 3, -1, -2, -3, 4, -4]
    assert per32[0] == 127 and q80[0] == 127


def test_zero_block_and_nan():
    x = np.zeros((1, 256), np.float32)
    for fmt in (O.ACT_PER32, O.ACT_Q8_0, O.ACT_Q8_K):
        assert not O.quantize_act(fmt, x).any()
    x[0, 3] = np.nan
    x[0, 4] = 2.0
    a = O.quantize_act(O.ACT_PER32, x)[0]
    assert a[:4].view(np.float32)[0] == np.float32(2.0) / np.float32(127.0)  # NaN never becomes amax
    assert a[8 + 3].view(np.int8) == -127                                    # the clamp sends NaN to -127


# ------------------------------------------------------------- dequantize


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_dequantize_golden(gold, t):
    name = O.TYPE_NAMES[t]
    mine = O.dequantize(t, gold[f"w_{name}"], 512)
    assert np.array_equal(mine.view(np.uint32), gold[f"deq_{name}"].view(np.uint32))


def test_dequantize_closed_forms():
    """Hand-built blocks with known values."""
    # Q8_0: d = 0.5 (fp16 0x3800), codes 0..31 -> 0.5 * i
    b = np.zeros(34, np.uint8)
    b[0:2] = np.array([0x3800], np.uint16).view(np.uint8)
    b[2:] = np.arange(32, dtype=np.int8).view(np.uint8)
    assert np.array_equal(O.dequantize(O.Q8_0, b, 32)[0], 0.5 * np.arange(32, dtype=np.float32))
    # Q4_0: d = 1, nibbles lo = i % 16 -> value (i - 8), hi -> element 16 + i
    b = np.zeros(18, np.uint8)
    b[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)
    b[2:] = (np.arange(16) | ((15 - np.arange(16)) << 4)).astype(np.uint8)
    want = np.concatenate([np.arange(16) - 8, (15 - np.arange(16)) - 8]).astype(np.float32)
    assert np.array_equal(O.dequantize(O.Q4_0, b, 32)[0], want)
    # Q4_K: d = 1, dmin = 1, sc_j = j + 1, m_j = 2j, all codes 3 -> (j+1)*3 - 2j
    b = np.zeros(144, np.uint8)
    b[0:4] = np.array([0x3C00, 0x3C00], np.uint16).view(np.uint8)
    sc = [j + 1 for j in range(8)]
    mn = [2 * j for j in range(8)]
    for j in range(4):
        b[4 + j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        b[8 + j] = mn[j] | ((mn[j + 4] >> 4) << 6)
        b[12 + j] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    b[16:] = 0x33
    want = np.repeat([3 * sc[j] - mn[j] for j in range(8)], 32).astype(np.float32)
    assert np.array_equal(O.dequantize(O.Q4_K, b, 256)[0], want)
    # Q6_K: d = 1, scales = 1; value e has 6-bit code e % 64 -> e % 64 - 32
    codes = np.arange(256) % 64
    b = np.zeros(210, np.uint8)
    for p in range(2):
        v = codes[128 * p:128 * p + 128]
        for l in range(32):
            b[64 * p + l] = (v[l] & 15) | ((v[l + 64] & 15) << 4)
            b[64 * p + l + 32] = (v[l + 32] & 15) | ((v[l + 96] & 15) << 4)
            b[128 + 32 * p + l] = (v[l] >> 4) | ((v[l + 32] >> 4) << 2) | ((v[l + 64] >> 4) << 4) | ((v[l + 96] >> 4) << 6)
    b[192:208] = 1
    b[208:210] = np.array([0x3C00], np.uint16).view(np.uint8)
    assert np.array_equal(O.dequantize(O.Q6_K, b, 256)[0], (codes - 32).astype(np.float32))


# ---------------------------------------------------------------- partials


def _int_codes(t: int, w: np.ndarray, k: int) -> np.ndarray:
    """Integer weight codes recovered through the dequantizer with d = 1, dmin = 0
    and unit scales (the reference's own dequantizer where oracle/_ref exists)."""
    w = w.copy()
    be, bb = BLOCK[t]
    one = np.array([0x3C00], np.uint16).view(np.uint8)
    for b in range(k // be):
        o = b * bb
        if t in (O.Q8_0, O.Q4_0):
            w[:, o:o + 2] = one
        elif t == O.Q4_K:
            w[:, o:o + 2] = one
            w[:, o + 2:o + 4] = 0
            w[:, o + 4:o + 16] = np.array([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1], np.uint8)
        else:
            w[:, o + 192:o + 208] = 1
            w[:, o + 208:o + 210] = one
    if O.ref_available():
        deq = np.stack([O.ref_dequantize(t, w[i], k) for i in range(w.shape[0])])
    else:
        deq = O.dequantize(t, w, k)
    codes = deq.astype(np.int64)
    assert np.array_equal(codes.astype(np.float32), deq)
    return codes


def _act_codes(fmt: int, a: np.ndarray, k: int) -> np.ndarray:
    if fmt == O.ACT_PER32:
        return a.reshape(a.shape[0], -1, 40)[:, :, 8:].view(np.int8).reshape(a.shape[0], k).astype(np.int64)
    if fmt == O.ACT_Q8_0:
        return a.reshape(a.shape[0], -1, 34)[:, :, 2:].view(np.int8).reshape(a.shape[0], k).astype(np.int64)
    if fmt == O.ACT_Q8_K:
        return a.reshape(a.shape[0], -1, 292)[:, :, 4:260].view(np.int8).reshape(a.shape[0], k).astype(np.int64)
    if fmt == O.ACT_Q16:
        return a.reshape(a.shape[0], -1, 72)[:, :, 8:].copy().view(np.int16).reshape(a.shape[0], k).astype(np.int64)
    return a.reshape(a.shape[0], -1, 320)[:, :, :256].view(np.int8).reshape(a.shape[0], k).astype(np.int64)


PAIRS_ALL = [(O.Q8_0, O.ACT_PER32), (O.Q8_0, O.ACT_Q8_0), (O.Q4_0, O.ACT_PER32), (O.Q4_0, O.ACT_Q8_0),
             (O.Q4_K, O.ACT_PER32), (O.Q4_K, O.ACT_Q8_K), (O.Q4_K, O.ACT_SX),
             (O.Q6_K, O.ACT_PER32), (O.Q6_K, O.ACT_Q8_K), (O.Q6_K, O.ACT_SX),
             (O.Q8_0, O.ACT_Q16), (O.Q4_0, O.ACT_Q16), (O.Q4_K, O.ACT_Q16), (O.Q6_K, O.ACT_Q16)]


@pytest.mark.parametrize("t,fmt", PAIRS_ALL, ids=lambda p: str(p))
def test_partials_brute_force(t, fmt):
    k = 512
    w = weight_rows(t, 3, k, 77 + t, edge=True)
    x = activations(2, k, 78)
    a = O.quantize_act(fmt, x)
    units, sb = O.partials(t, fmt, w, a, k)
    wc = _int_codes(t, w, k)
    ac = _act_codes(fmt, a, k)
    ul = 16 if t == O.Q6_K else 32
    prod = (ac[:, None, :] * wc[None, :, :]).reshape(2, 3, k // ul, ul).sum(-1)
    assert np.array_equal(units, prod)
    if sb.shape[-1]:
        nsb = k // 256
        for n in range(3):
            for b in range(nsb):
                blk = w[n, b * BLOCK[t][1]:(b + 1) * BLOCK[t][1]]
                if t == O.Q4_K:
                    scm = [_scale_min_bitfields(bytes(blk[4:16]), j) for j in range(8)]
                    scale = [s for s, _ in scm]
                    mins = [mm for _, mm in scm]
                else:
                    scale = list(blk[192:208].view(np.int8).astype(int))
                    mins = [0] * 16
                for r in range(2):
                    mult = [1] * 8
                    if fmt == O.ACT_SX:
                        mult = list(a[r, b * 320 + 260:b * 320 + 276].copy().view(np.int16))
                    nunit = 256 // ul
                    S = sum(int(scale[u]) * int(mult[u * ul // 32]) * int(prod[r, n, b * nunit + u]) for u in range(nunit))
                    sums = ac[r, b * 256:(b + 1) * 256].reshape(8, 32).sum(-1)
                    Mn = sum(int(mins[j]) * int(mult[j]) * int(sums[j]) for j in range(8))
                    if fmt == O.ACT_SX:  # S in 64 bits: low and high words, then Mn
                        got = (int(sb[r, n, 3 * b + 1]) << 32) | (int(sb[r, n, 3 * b]) & 0xFFFFFFFF)
                        assert got == S
                        if t == O.Q4_K:
                            assert sb[r, n, 3 * b + 2] == Mn
                    else:
                        assert sb[r, n, 2 * b] == S
                        if t == O.Q4_K:
                            assert sb[r, n, 2 * b + 1] == Mn


# -------------------------------------------------------------------- dots


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_generic_dots_golden_bit_exact(gold, t):
    name = O.TYPE_NAMES[t]
    y = O.matmul(t, O.ACT_PER32, gold[f"w_{name}"], gold["act_per32"], 512)
    assert np.array_equal(y.view(np.uint32), gold[f"dot_{name}"].view(np.uint32))


@pytest.mark.parametrize("t", (O.Q4_K, O.Q6_K), ids=lambda t: O.TYPE_NAMES[t])
def test_q8K_and_sx_dots_vs_reference_avx2(gold, t):
    """Q8_K (canonical order) vs the reference super-block kernel on the same codes,
    and sub-scaled vs the reference sx kernel: fp32 reorderings only, so every output
    is held to a per-element bound on its own sum of |terms|: 1e-6 of it, a tenth of
    the reference's (test_int_kernels.cpp:131-147; the two orders differ by at most
    2e-8 of it on these vectors, while one dropped or doubled term moves an output by
    ~1/512 of it)."""
    name = O.TYPE_NAMES[t]
    w = gold[f"w_{name}"]
    wf = np.abs(O.dequantize(t, w, 512).astype(np.float64))
    aq = O.quantize_act(O.ACT_Q8_K, gold["act_x"])
    yq = O.matmul(t, O.ACT_Q8_K, w, aq, 512)
    mag = np.abs(O.dequantize_act(O.ACT_Q8_K, aq, 512).astype(np.float64)) @ wf.T
    assert np.all(np.isfinite(mag))
    assert np.all(np.abs(yq - gold[f"sbdot_{name}"]) <= 1e-6 * mag)
    ys = O.matmul(t, O.ACT_SX, w, gold["act_sx"], 512)
    mag_s = np.abs(O.dequantize_act(O.ACT_SX, gold["act_sx"], 512).astype(np.float64)) @ wf.T
    assert np.all(np.abs(ys - gold[f"sxdot_{name}"]) <= 1e-6 * mag_s)


@pytest.mark.parametrize("t", (O.Q8_0, O.Q4_K, O.Q6_K), ids=lambda t: O.TYPE_NAMES[t])
def test_q16_dots_vs_reference_avx2(gold, t):
    """int16 dots vs the reference's AVX2 dot_rows16_* on the same bytes: the same
    exact integers, fp32 lane order only (1e-5 of the sum of |terms|,
    test_int_kernels.cpp:181-193); the edge row included."""
    name = O.TYPE_NAMES[t]
    w = gold[f"w_{name}"]
    a = gold["act_q16"]
    y = O.matmul(t, O.ACT_Q16, w, a, 512)
    mag = np.abs(O.dequantize_act(O.ACT_Q16, a, 512).astype(np.float64)) @ np.abs(O.dequantize(t, w, 512).astype(np.float64)).T
    fin = np.isfinite(mag)
    assert fin[:4].all()
    assert np.all(np.abs(y - gold[f"q16dot_{name}"])[fin] <= 1e-5 * mag[fin])
    # the edge row holds +-inf inputs (a block with d = inf): no finite result on either
    # side; whether inf or NaN depends on how the products are grouped (the reference's
    # 8 lanes give 0 * inf = NaN in lanes without the inf's code)
    assert not np.isfinite(y[4]).any() and not np.isfinite(gold[f"q16dot_{name}"][4]).any()


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_f32_dots_golden_bit_exact(gold, t):
    """fp32 activations (the kF32 contract): bit-equal to the reference's generic vec_dot_*."""
    name = O.TYPE_NAMES[t]
    y = O.matmul(t, O.ACT_F32, gold[f"w_{name}"], O.quantize_act(O.ACT_F32, gold["act_x"]), 512)
    assert np.array_equal(y.view(np.uint32), gold[f"vecdot_{name}"].view(np.uint32))


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_f32_dots_within_double_bound(t):
    """The fp32 dots against the double product of the dequantized weights and the fp32
    rows: 1e-5 of the sum of |terms| (edge weight blocks, outlier channels)."""
    k = 1024
    w = weight_rows(t, 5, k, 320 + t, edge=True)
    x = activations(3, k, 321)
    y = O.matmul(t, O.ACT_F32, w, O.quantize_act(O.ACT_F32, x), k)
    wf = O.dequantize(t, w, k).astype(np.float64)
    xf = x.astype(np.float64)
    assert np.all(np.abs(y - xf @ wf.T) <= 1e-5 * (np.abs(xf) @ np.abs(wf).T) + 1e-30)
    assert np.array_equal(O.dequantize_act(O.ACT_F32, O.quantize_act(O.ACT_F32, x), k), x)


@pytest.mark.parametrize("t,fmt", PAIRS_ALL, ids=lambda p: str(p))
def test_dots_within_double_bound(t, fmt):
    """|y - y_double| <= 1e-5 * sum|w_i x_i| against the double product of the
    dequantized weights and activations (test_int_kernels.cpp:131-147)."""
    k = 1024
    w = weight_rows(t, 5, k, 300 + t, edge=True)
    x = activations(3, k, 301)
    a = O.quantize_act(fmt, x)
    y = O.matmul(t, fmt, w, a, k)
    wf = O.dequantize(t, w, k).astype(np.float64)
    af = O.dequantize_act(fmt, a, k).astype(np.float64)
    ref = af @ wf.T
    mag = np.abs(af) @ np.abs(wf).T
    assert np.all(np.abs(y - ref) <= 1e-5 * mag + 1e-30)


# ---------------------------------------------------------------- encoders


@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_encoders_error_bound(t):
    k = 2048
    x = O.normal(9, 4 * k, std=0.02, outlier_frac=0.01, outlier_sigma=8.0).reshape(4, k)
    w = O.encode_weight(t, x)
    xr = O.dequantize(t, w, k)
    be = BLOCK[t][0]
    err = np.abs(xr - x).reshape(4, -1, 32 if t != O.Q6_K else 16)
    span = np.abs(x).reshape(err.shape).max(-1, keepdims=True)
    # Q4_K: 15 steps over [min(0, lo), hi] (<= 2 span), half a step of error plus the
    # rounding of the 6-bit scale and offset (ceil) to the super-block grid; Q6_K: step
    # span/31; Q8_0: step span/127. Q4_0 maps the largest magnitude to code -8, so the
    # other side clamps at +7 steps of span/8: up to one full step there.
    # (Q8_0 codes use the fp32 d but decode with its fp16 rounding: + 127 * 2^-11 steps)
    bound = {O.Q8_0: (0.5 + 127 * 2.0**-11) / 127.0, O.Q4_0: 1.0 / 8.0, O.Q4_K: 0.6 * 2.0 / 15.0, O.Q6_K: 0.5 / 31.0}[t]
    if t == O.Q6_K:
        # Q6_K codes never clamp (|x| / step <= 31): half of the unit's own step d * sc
        blk = w.reshape(4, -1, 210)
        d = O.fp16_to_fp32(blk[:, :, 208:210].copy().view(np.uint16)[..., 0]).astype(np.float64)
        st = d[..., None] * blk[:, :, 192:208].view(np.int8).astype(np.float64)
        assert np.all(err <= 0.5 * st.reshape(err.shape[:2])[..., None] * (1 + 1e-3) + 1e-9)
    else:
        assert np.all(err <= bound * span * (1 + 5e-3) + 1e-7), be
    if O.ref_available():
        ref = np.stack([O.ref_dequantize(t, w[i], k) for i in range(4)])
        assert np.array_equal(ref.view(np.uint32), xr.view(np.uint32))


# ------------------------------------------------------------ live reference


@needs_ref
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_live_reference_quantizers(seed):
    x = activations(3, 2048, seed)
    for kind, fmt in (("q8_0", O.ACT_Q8_0), ("per32", O.ACT_PER32), ("per32_avx2", O.ACT_PER32), ("sx", O.ACT_SX),
                      ("q16", O.ACT_Q16)):
        ref = np.stack([O.ref_quantize(kind, x[i]) for i in range(3)])
        assert np.array_equal(O.quantize_act(fmt, x), ref), kind


@needs_ref
@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_live_reference_vec_dot(t):
    """fp32 activations: generic vec_dot bit-equal, AVX2 vec_dot within its fp32 reordering."""
    k = 2048
    w = weight_rows(t, 4, k, 520 + t, edge=True)
    x = activations(3, k, 521)
    y = O.matmul(t, O.ACT_F32, w, O.quantize_act(O.ACT_F32, x), k)
    gen = np.array([[O.ref_vec_dot(0, t, w[i], x[r], k) for i in range(4)] for r in range(3)], np.float32)
    avx = np.array([[O.ref_vec_dot(1, t, w[i], x[r], k) for i in range(4)] for r in range(3)], np.float32)
    assert np.array_equal(y.view(np.uint32), gen.view(np.uint32))
    mag = np.abs(x.astype(np.float64)) @ np.abs(O.dequantize(t, w, k).astype(np.float64)).T
    assert np.all(np.abs(avx - y) <= 1e-5 * mag)


@needs_ref
@pytest.mark.parametrize("t", TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_live_reference_generic_dots(t):
    k = 2048
    w = weight_rows(t, 6, k, 500 + t, edge=True)
    a = O.quantize_act(O.ACT_PER32, activations(4, k, 501))
    y = O.matmul(t, O.ACT_PER32, w, a, k)
    ref = np.stack([O.ref_dot_rows(0, t, w[i], a, k) for i in range(6)], 1)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


# ----------------------------------------------------------- activations


def test_exp_nonpos_golden(gold):
    """Bit-equal to the reference's exp_nonpos (base/fast_exp.h:16-35), boundary and NaN inputs included."""
    y = O.exp_nonpos(gold["expnp_x"])
    assert np.array_equal(y.view(np.uint32), gold["expnp_y"].view(np.uint32))


def test_exp_nonpos_vs_double_exp():
    x = np.concatenate([np.linspace(-87.0, 0.0, 20001), -np.random.default_rng(5).exponential(3.0, 20000)])
    x = x[x >= -87.0].astype(np.float32)
    y = O.exp_nonpos(x).astype(np.float64)
    ex = np.exp(x.astype(np.float64))
    assert np.max(np.abs(y - ex) / ex) < 3e-7
    assert O.exp_nonpos(np.array([0.0], np.float32))[0] == 1.0
    # clamp: below -87 (and NaN, -inf) the value at -87
    lo = O.exp_nonpos(np.array([-87.0, -88.0, -1e9, -np.inf, np.nan], np.float32))
    assert np.all(lo == lo[0]) and abs(lo[0] / np.exp(-87.0) - 1) < 3e-7


def _act_double(act: int, x: np.ndarray) -> np.ndarray:
    import math
    xd = x.astype(np.float64)
    if act == O.SILU:
        return xd / (1.0 + np.exp(-xd))
    if act == O.GELU:
        return 0.5 * xd * (1.0 + np.array([math.erf(v / math.sqrt(2.0)) for v in xd]))
    return 0.5 * xd * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (xd + 0.044715 * xd ** 3)))


@pytest.mark.parametrize("act", [O.SILU, O.GELU, O.GELU_TANH], ids=["silu", "gelu", "gelu_tanh"])
def test_activations_closed_forms(act):
    """Within fp32 rounding of the textbook forms: SiLU x sigmoid(x); GELU with erf; GELU's tanh form
    (cpu_device.cpp:117-128)."""
    rng = np.random.default_rng(7 + act)
    x = np.concatenate([rng.normal(0.0, 4.0, 20000), np.linspace(-30.0, 30.0, 6001), [0.0, -0.0, 1e-30, -1e-30]])
    x = x.astype(np.float32)
    y = O.activation(act, x)
    ref = _act_double(act, x)
    scale = np.maximum(np.abs(x.astype(np.float64)), 1.0)
    bound = 3e-7 if act == O.SILU else 2.5e-7
    assert np.max(np.abs(y - ref) / scale) < bound
    if act == O.SILU:  # the exponential is exp_nonpos: relative accuracy holds down to the clamp
        keep = np.abs(ref) > 1e-30
        assert np.max(np.abs(y[keep] - ref[keep]) / np.abs(ref[keep])) < 5e-7
    big = np.array([40.0, 1000.0], np.float32)
    assert np.array_equal(O.activation(act, big), big)
    assert O.activation(act, np.array([0.0], np.float32))[0] == 0.0


def test_silu_rounding_sequence(gold):
    """SiLU's fp32 sequence x * (x >= 0 ? 1 : e) / (1 + e) on the reference's own e^-|x| values: each
    step one IEEE rounding, so numpy float32 steps on the golden exponentials give the same bits."""
    e_in = gold["expnp_x"]
    sel = np.isfinite(e_in) & (e_in <= 0) & (e_in >= -87)
    e = gold["expnp_y"][sel]
    mag = -e_in[sel]
    for sign in (1.0, -1.0):
        x = (np.float32(sign) * mag).astype(np.float32)
        num = np.where(x >= 0, np.float32(1.0), e).astype(np.float32)
        want = ((x * num).astype(np.float32) / (np.float32(1.0) + e).astype(np.float32)).astype(np.float32)
        got = O.activation(O.SILU, x)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_activation_rejects_unknown():
    with pytest.raises(ValueError):
        O.activation(3, np.zeros(4, np.float32))


@pytest.mark.parametrize("act", [O.SILU, O.GELU, O.GELU_TANH], ids=["silu", "gelu", "gelu_tanh"])
def test_matmul_gated_vs_double(act):
    """act(x . Wg^T) * (x . Wu^T) against double-precision dots of the dequantized operands."""
    k, n = 512, 12
    wg = weight_rows(O.Q4_K, n, k, 61)
    wu = weight_rows(O.Q6_K, n, k, 62)
    a = O.quantize_act(O.ACT_Q8_K, activations(3, k, 63))
    y = O.matmul_gated(act, O.Q4_K, O.Q6_K, O.ACT_Q8_K, wg, wu, a, k)
    xa = np.stack([O.dequantize_act(O.ACT_Q8_K, a[i], k).ravel() for i in range(3)]).astype(np.float64)
    g = xa @ np.stack([O.dequantize(O.Q4_K, wg[i], k).ravel() for i in range(n)]).astype(np.float64).T
    u = xa @ np.stack([O.dequantize(O.Q6_K, wu[i], k).ravel() for i in range(n)]).astype(np.float64).T
    ref = _act_double(act, g.astype(np.float32).ravel()).reshape(g.shape) * u
    scale = np.maximum(np.abs(g), 1.0) * np.maximum(np.abs(u), 1.0)
    assert np.max(np.abs(y - ref) / scale) < 1e-4


def _q4k_extreme_row(k: int) -> np.ndarray:
    """Q4_K row with every scale 63, every min 0, every code 15 and d = 1: the largest S."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[4:8] = 0xFF      # sc_0..3 = 63 and the top bits of sc_4..7
    blk[12:16] = 0x0F    # low bits of sc_4..7 (mins stay 0)
    blk[16:] = 0xFF
    return np.tile(blk, k // 256)[None, :]


def test_subscaled_s_exceeds_int32():
    """Sub-scaled S = sum sc * m_b * P exceeds 2^31 for constant inputs and extreme weights; the
    oracle keeps it exact (64 bits) and the dot matches the double product."""
    k = 256
    w = _q4k_extreme_row(k)
    assert [_scale_min_bitfields(bytes(w[0, 4:16]), j) for j in range(8)] == [(63, 0)] * 8
    x = np.full((1, k), 3.0, np.float32)
    a = O.quantize_act(O.ACT_SX, x)
    assert np.all(a[0, 260:276].view(np.int16) == 128) and np.all(a[0, :256].view(np.int8) == 127)
    _, sb = O.partials(O.Q4_K, O.ACT_SX, w, a, k)
    S = (int(sb[0, 0, 1]) << 32) | (int(sb[0, 0, 0]) & 0xFFFFFFFF)
    assert S == 8 * 63 * 128 * 32 * 15 * 127 > 2 ** 31
    y = O.matmul(O.Q4_K, O.ACT_SX, w, a, k)
    ref = float(O.dequantize_act(O.ACT_SX, a, k).astype(np.float64) @ O.dequantize(O.Q4_K, w[0], k).ravel())
    assert abs(float(y[0, 0]) - ref) <= 1e-6 * abs(ref)


# ---------------------------------------------------------------- qmm activation buffer

def _qmm_rows(m: int, k: int, seed: int) -> np.ndarray:
    """Rows of N(0, 3) with the cases the reference's clamp and rounding decide: NaN, +-Inf,
    all-zero and negative-zero blocks, half-way codes, a block whose amax is exactly qmax."""
    x = (np.random.default_rng(seed).standard_normal((m, k)) * 3).astype(np.float32)
    x[0, 3] = np.nan
    x[m - 1, min(40, k - 1)] = np.inf
    if k >= 128:
        x[0, 64:96] = 0.0
        x[0, 96:128] = -0.0
        x[m - 1, 0] = -np.inf
    if k >= 64:
        x[m - 1, 32] = 127.0
        x[m - 1, 33:64] = np.float32(0.5) + np.arange(31, dtype=np.float32)  # codes at exact .5 ties
    return x


@needs_ref
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("paired", [False, True])
@pytest.mark.parametrize("m,k", [(1, 32), (2, 256), (3, 1536), (8, 4096)])
def test_qmm_quantize_matches_reference(mode, paired, m, k):
    """The oracle's qmm buffer is byte-identical to the reference's own ActBuffer filled by
    its reference tier (dynacore/cpu/qmm/qmm_reference.cpp:25-51,440-488, built in oracle/_ref)."""
    x = _qmm_rows(m, k, 11 * m + k)
    got, want = O.qmm_quantize(x, mode, paired), O.ref_qmm_quantize(x, mode, paired)
    for g, w in zip(got, want):
        assert (g is None) == (w is None)
        if g is not None:
            assert g.tobytes() == w.tobytes()


@pytest.mark.parametrize("mode", [0, 1])
def test_qmm_quantize_layouts_and_scales(mode):
    """Without the reference: the pair layout is the row layout interleaved in 8-byte chunks
    (qmm.h:63-66), the pad row of an odd m is zero, c = d * (code sum) per block, codes stay
    within +-qmax and a block's largest |x| maps to +-qmax."""
    m, k = 5, 512
    x = (np.random.default_rng(5).standard_normal((m, k)) * 2).astype(np.float32)
    hi_r, lo_r, d_r, c_r = O.qmm_quantize(x, mode, False)
    hi_p, lo_p, d_p, c_p = O.qmm_quantize(x, mode, True)
    kb, qmax = k // 32, (127 if mode == 0 else 32767)
    q = hi_r.astype(np.int32) if mode == 0 else hi_r.astype(np.int32) * 256 + lo_r.astype(np.int32)
    q = q.reshape(m, k)
    assert np.abs(q).max() <= qmax
    sums = q.reshape(m, kb, 32).sum(axis=2)
    np.testing.assert_array_equal(c_r.reshape(m, kb), (d_r.reshape(m, kb) * sums.astype(np.float32)).astype(np.float32))
    big = np.abs(x.reshape(m, kb, 32)).argmax(axis=2)
    assert (np.abs(np.take_along_axis(q.reshape(m, kb, 32), big[..., None], 2)) == qmax).all()
    m_pad = m + 1
    inter = np.zeros((m_pad // 2, k // 8, 2, 8), np.int8)
    rows = np.zeros((m_pad, k), np.int8)
    rows[:m] = hi_r.reshape(m, k)
    inter[:, :, 0] = rows[0::2].reshape(m_pad // 2, k // 8, 8)
    inter[:, :, 1] = rows[1::2].reshape(m_pad // 2, k // 8, 8)
    assert hi_p.tobytes() == inter.tobytes()
    dd = np.zeros((m_pad, kb), np.float32)
    dd[:m] = d_r.reshape(m, kb)
    np.testing.assert_array_equal(d_p.reshape(m_pad // 2, kb, 2), np.stack([dd[0::2], dd[1::2]], axis=2))


def _q16_rows_from_qmm(x: np.ndarray) -> np.ndarray:
    """The rows of qmm's int16 buffer (row layout) as int16 activation blocks (float d,
    int32 code sum, int16 codes[32]): the conversion dq_qmm_gemv makes on the GPU."""
    hi, lo, d, _ = O.qmm_quantize(x, 1, False)
    m, k = x.shape
    kb = k // 32
    codes = (hi.astype(np.int32).reshape(m, kb, 32) * 256 + lo.astype(np.int32).reshape(m, kb, 32)).astype(np.int16)
    out = np.zeros((m, kb, 72), np.uint8)
    out[:, :, 0:4] = np.ascontiguousarray(d, np.float32).reshape(m, kb, 1).view(np.uint8)
    out[:, :, 4:8] = codes.astype(np.int32).sum(-1, dtype=np.int32).reshape(m, kb, 1).view(np.uint8)
    out[:, :, 8:] = codes.view(np.uint8).reshape(m, kb, 64)
    return out.reshape(m, -1)


@needs_ref
def test_q16_q4_0_matches_reference_qmm():
    """Q4_0 x int16 has no AVX2 kernel in the reference; the oracle follows qmm's
    dot_row_ref (dynacore/cpu/qmm/qmm_reference.cpp:68-93, codes from qmm_unpack.h:61-75):
    on the reference's own int16 ActBuffer rows it equals the reference build's qmm gemv
    bit for bit (one accumulator, blocks in order, (dw * da) * P)."""
    m, k, n = 5, 1024, 40
    w = gguf_weights(O.Q4_0, n, k, 2100, outlier_frac=0.01)
    x = (np.random.default_rng(2101).standard_normal((m, k)) * 3).astype(np.float32)
    x[:, 5::67] *= np.float32(90.0)
    a16 = _q16_rows_from_qmm(x)
    got = O.matmul(O.Q4_0, O.ACT_Q16, w, a16, k)
    want = O.ref_qmm_gemv(O.Q4_0, w, x, 1, False)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_qmm_quantize_golden():
    """The oracle against the committed reference buffers (tests/golden/make_qmm_golden.py):
    both modes and layouts, 3 rows (a pad row when paired), NaN / Inf / zero / tie inputs."""
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qmm_vectors.npz"))
    for mode in (0, 1):
        for paired in (0, 1):
            key = f"m{mode}p{paired}"
            hi, lo, d, c = O.qmm_quantize(g["x"], mode, bool(paired))
            assert hi.tobytes() == g[f"{key}_hi"].tobytes()
            assert d.tobytes() == g[f"{key}_d"].tobytes() and c.tobytes() == g[f"{key}_c"].tobytes()
            assert (lo is None) == (mode == 0)
            if lo is not None:
                assert lo.tobytes() == g[f"{key}_lo"].tobytes()
