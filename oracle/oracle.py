"""ctypes bindings for the CPU oracle (liboracle.so) and the reference build (_ref).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by
bench.py's cpu_baseline leg, as the checker. The product (dynalm_amd) never
imports this module.

All functions take and return numpy arrays. Type ids are dynacore DType values
(dynacore/include/dynacore/tensor/dtype.h:19-44); activation format ids are the
DQO_ACT_* values of dq_oracle.h.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libdynacore_ref.so")

Q4_0, Q8_0, Q4_K, Q6_K, Q8_K = 6, 10, 14, 16, 17
ACT_PER32, ACT_Q8_0, ACT_Q8_K, ACT_SX, ACT_Q16, ACT_F32 = 0, 1, 2, 3, 4, 5
TYPE_NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_K", Q6_K: "q6_K", Q8_K: "q8_K"}
ACT_NAMES = {ACT_PER32: "per32", ACT_Q8_0: "q8_0", ACT_Q8_K: "q8_K", ACT_SX: "sx", ACT_Q16: "q16", ACT_F32: "f32"}

_P = C.c_void_p
_I64 = C.c_int64


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _load_oracle():
    lib = C.CDLL(ORACLE_SO)
    sig = {
        "dqo_block_elems": (_I64, [C.c_int]),
        "dqo_block_bytes": (_I64, [C.c_int]),
        "dqo_row_bytes": (_I64, [C.c_int, _I64]),
        "dqo_act_block_elems": (_I64, [C.c_int]),
        "dqo_act_row_bytes": (_I64, [C.c_int, _I64]),
        "dqo_fp16_to_fp32_n": (None, [_P, _P, _I64]),
        "dqo_fp32_to_fp16_n": (None, [_P, _P, _I64]),
        "dqo_scale_min_k4": (None, [C.c_int, _P, _P, _P]),
        "dqo_dequantize": (C.c_int, [C.c_int, _P, _P, _I64]),
        "dqo_expand_x86": (C.c_int, [C.c_int, _P, _P, _I64]),
        "dqo_dequantize_act": (C.c_int, [C.c_int, _P, _P, _I64]),
        "dqo_quantize_act": (C.c_int, [C.c_int, _P, _P, _I64]),
        "dqo_quantize_act_rows": (C.c_int, [C.c_int, _P, _I64, _I64, _I64, _P]),
        "dqo_qmm_quantize": (C.c_int, [_P, _I64, _I64, _I64, C.c_int, C.c_int, _P, _P, _P, _P]),
        "dqo_encode_weight": (C.c_int, [C.c_int, _P, _P, _I64]),
        "dqo_encode_weight_rows": (C.c_int, [C.c_int, _P, _I64, _I64, _P]),
        "dqo_partials_count": (C.c_int, [C.c_int, C.c_int, _I64, C.POINTER(_I64), C.POINTER(_I64)]),
        "dqo_partials": (C.c_int, [C.c_int, C.c_int, _P, _P, _I64, _P, _P]),
        "dqo_dot": (C.c_float, [C.c_int, C.c_int, _P, _P, _I64]),
        "dqo_matmul": (C.c_int, [C.c_int, C.c_int, _P, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _P]),
        "dqo_fill_normal": (None, [C.c_uint64, _P, _I64, C.c_double, C.c_double, C.c_double, C.c_double]),
        "dqo_fill_bytes": (None, [C.c_uint64, _P, _I64]),
        "dqo_exp_nonpos": (C.c_float, [C.c_float]),
        "dqo_activation": (C.c_int, [C.c_int, _P, _P, _I64]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} is not built (make -C oracle)")
        _lib = _load_oracle()
    return _lib


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what} failed ({rc})")


# ------------------------------------------------------------------ sizes


def row_bytes(dtype: int, k: int) -> int:
    return int(lib().dqo_row_bytes(dtype, k))


def act_row_bytes(fmt: int, k: int) -> int:
    return int(lib().dqo_act_row_bytes(fmt, k))


# ------------------------------------------------------------------- fp16


def fp16_to_fp32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().dqo_fp16_to_fp32_n(_ptr(h), _ptr(out), h.size)
    return out


def fp32_to_fp16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().dqo_fp32_to_fp16_n(_ptr(f), _ptr(out), f.size)
    return out


# ------------------------------------------------------------------ inputs


def normal(seed: int, n: int, mean=0.0, std=1.0, outlier_frac=0.0, outlier_sigma=0.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().dqo_fill_normal(seed & (2**64 - 1), _ptr(out), n, mean, std, outlier_frac, outlier_sigma)
    return out


def random_bytes(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint8)
    lib().dqo_fill_bytes(seed & (2**64 - 1), _ptr(out), n)
    return out


# ---------------------------------------------------------- quant formats


def encode_weight(dtype: int, x: np.ndarray) -> np.ndarray:
    """x: [rows, k] fp32 -> [rows, row_bytes] uint8 GGUF blocks."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    rows, k = x.shape
    out = np.empty((rows, row_bytes(dtype, k)), np.uint8)
    _check(lib().dqo_encode_weight_rows(dtype, _ptr(x), rows, k, _ptr(out)), "encode_weight")
    return out


def dequantize(dtype: int, blocks: np.ndarray, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(np.atleast_2d(blocks), dtype=np.uint8)
    rows = blocks.shape[0]
    out = np.empty((rows, k), np.float32)
    for r in range(rows):
        _check(lib().dqo_dequantize(dtype, _ptr(blocks[r]), _ptr(out[r]), k), "dequantize")
    return out


def expand_x86(dtype: int, blocks: np.ndarray, k: int) -> np.ndarray:
    """The fp32 expand + GEMM class's weight expansion (one fma per value, the
    reference's x86 dequant), [rows, k]."""
    blocks = np.ascontiguousarray(np.atleast_2d(blocks), dtype=np.uint8)
    out = np.empty((blocks.shape[0], k), np.float32)
    for r in range(blocks.shape[0]):
        _check(lib().dqo_expand_x86(dtype, _ptr(blocks[r]), _ptr(out[r]), k), "expand_x86")
    return out


def quantize_act(fmt: int, x: np.ndarray) -> np.ndarray:
    """x: [m, k] fp32 -> [m, act_row_bytes] uint8."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    m, k = x.shape
    out = np.empty((m, act_row_bytes(fmt, k)), np.uint8)
    _check(lib().dqo_quantize_act_rows(fmt, _ptr(x), m, k, k, _ptr(out)), "quantize_act")
    return out


def dequantize_act(fmt: int, a: np.ndarray, k: int) -> np.ndarray:
    a = np.ascontiguousarray(np.atleast_2d(a), dtype=np.uint8)
    out = np.empty((a.shape[0], k), np.float32)
    for r in range(a.shape[0]):
        _check(lib().dqo_dequantize_act(fmt, _ptr(a[r]), _ptr(out[r]), k), "dequantize_act")
    return out


def partials_count(wtype: int, fmt: int, k: int):
    u, s = _I64(), _I64()
    _check(lib().dqo_partials_count(wtype, fmt, k, C.byref(u), C.byref(s)), "partials_count")
    return int(u.value), int(s.value)


def partials(wtype: int, fmt: int, w: np.ndarray, a: np.ndarray, k: int):
    """Integer partials for every (activation row r, weight row n):
    units [m, n, U] int32 and super-block terms [m, n, S] int32."""
    w = np.ascontiguousarray(np.atleast_2d(w), dtype=np.uint8)
    a = np.ascontiguousarray(np.atleast_2d(a), dtype=np.uint8)
    nu, ns = partials_count(wtype, fmt, k)
    units = np.zeros((a.shape[0], w.shape[0], nu), np.int32)
    sb = np.zeros((a.shape[0], w.shape[0], max(ns, 1)), np.int32)
    for r in range(a.shape[0]):
        for n in range(w.shape[0]):
            _check(lib().dqo_partials(wtype, fmt, _ptr(w[n]), _ptr(a[r]), k, _ptr(units[r, n]), _ptr(sb[r, n])),
                   "partials")
    return units, sb[:, :, :ns]


def matmul(wtype: int, fmt: int, w: np.ndarray, a: np.ndarray, k: int, bias: np.ndarray | None = None) -> np.ndarray:
    """y[m, n] = dot(weight row n, act row m) (+ bias[n]), oracle order."""
    w = np.ascontiguousarray(np.atleast_2d(w), dtype=np.uint8)
    a = np.ascontiguousarray(np.atleast_2d(a), dtype=np.uint8)
    n, m = w.shape[0], a.shape[0]
    y = np.empty((m, n), np.float32)
    bp = None
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.float32)
        bp = _ptr(bias)
    _check(lib().dqo_matmul(wtype, fmt, _ptr(w), w.shape[1], n, _ptr(a), a.shape[1], m, k, _ptr(y), n, bp), "matmul")
    return y


# ------------------------------------------------------------ activations


SILU, GELU, GELU_TANH = 0, 1, 2


def exp_nonpos(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([lib().dqo_exp_nonpos(float(v)) for v in x], np.float32)


def activation(act: int, x: np.ndarray) -> np.ndarray:
    """act(x) elementwise (dynacore Activation: 0 SiLU, 1 GELU, 2 GELU-tanh)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    _check(lib().dqo_activation(act, _ptr(x), _ptr(y), x.size), "dqo_activation")
    return y


def matmul_gated(act: int, wt_gate: int, wt_up: int, fmt: int, w_gate: np.ndarray, w_up: np.ndarray, a: np.ndarray,
                 k: int) -> np.ndarray:
    """act(x . w_gate^T) * (x . w_up^T) on quantized activations a (Device::matmul_gated,
    dynacore/include/dynacore/device/device.h:188-199; the product in fp32)."""
    g = matmul(wt_gate, fmt, w_gate, a, k)
    u = matmul(wt_up, fmt, w_up, a, k)
    return (activation(act, g) * u).astype(np.float32)


# ------------------------------------------------------------ reference


_ref = None


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref():
    """The reference's own CPU kernels (oracle/_ref), or None when not built."""
    global _ref
    if _ref is None:
        if not ref_available():
            return None
        r = C.CDLL(REF_SO)
        sig = {
            "ref_has_avx2": (C.c_int, []),
            "ref_physical_cores": (C.c_int, []),
            "ref_logical_cores": (C.c_int, []),
            "ref_fp16_to_fp32": (C.c_float, [C.c_uint16]),
            "ref_fp32_to_fp16": (C.c_uint16, [C.c_float]),
            "ref_dequantize": (C.c_int, [C.c_int, _P, _P, _I64]),
            "ref_quantize_q8_0": (C.c_int, [_P, _P, _I64]),
            "ref_quantize_act": (C.c_int, [C.c_int, _P, _P, _I64]),
            "ref_quantize_act_sb": (C.c_int, [_P, _P, _I64]),
            "ref_quantize_act_sx": (C.c_int, [_P, _P, _I64]),
            "ref_dot_rows": (C.c_int, [C.c_int, C.c_int, _P, _P, _I64, C.c_int, _I64, _P]),
            "ref_dot_rows_n": (C.c_int, [C.c_int, C.c_int, _P, _I64, _I64, _I64, _P, _I64, C.c_int, _I64, _P, _I64, _P]),
            "ref_exp_nonpos": (C.c_float, [C.c_float]),
            "ref_quantize_act16": (C.c_int, [_P, _P, _I64]),
            "ref_split_act16": (C.c_int, [_P, _P, _I64]),
            "ref_dot_rows16": (C.c_int, [C.c_int, _P, _P, _I64, C.c_int, _I64, _P]),
            "ref_vec_dot": (C.c_int, [C.c_int, C.c_int, _P, _P, _I64, _P]),
            "ref_select_matmul": (C.c_int, [_I64, _I64, _I64, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                            C.c_int, C.c_int, C.c_uint32, C.c_int, C.c_int, C.POINTER(C.c_int)]),
            "ref_expand_x86": (C.c_int, [C.c_int, _P, _P, _I64]),
            "ref_qmm_quantize": (C.c_int, [_P, _I64, _I64, _I64, C.c_int, C.c_int, _P, _P, _P, _P]),
            "ref_qmm_gemv": (C.c_int, [C.c_int, _P, _I64, _I64, _P, _I64, _I64, C.c_int, C.c_int, _P]),
            "ref_bench_decode_sx": (_I64, [C.c_int, C.POINTER(_P), C.c_int, _I64, _I64, _P, C.c_int, _I64, _P,
                                           C.c_int, C.c_int, C.c_int]),
            "ref_llc_bytes": (_I64, []),
            "ref_expand_gemm": (C.c_int, [C.c_int, _P, _I64, _I64, _P, _I64, _I64, _P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(r, name)
            f.restype = res
            f.argtypes = args
        _ref = r
    return _ref


def ref_quantize(kind: str, x: np.ndarray) -> np.ndarray:
    """The reference's quantizers on one row: 'q8_0' (GGUF), 'per32' (generic),
    'per32_avx2', 'sb' (AVX2 super-block, ActBlockQ8 layout), 'sx' (AVX2), 'q16' (AVX2 int16)."""
    r = ref()
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    k = x.size
    if kind == "q8_0":
        out = np.empty(k // 32 * 34, np.uint8)
        _check(r.ref_quantize_q8_0(_ptr(x), _ptr(out), k), kind)
    elif kind in ("per32", "per32_avx2"):
        out = np.empty(k // 32 * 40, np.uint8)
        _check(r.ref_quantize_act(1 if kind == "per32_avx2" else 0, _ptr(x), _ptr(out), k), kind)
    elif kind == "sb":
        out = np.empty(k // 32 * 40, np.uint8)
        _check(r.ref_quantize_act_sb(_ptr(x), _ptr(out), k), kind)
    elif kind == "sx":
        out = np.empty(k // 256 * 320, np.uint8)
        _check(r.ref_quantize_act_sx(_ptr(x), _ptr(out), k), kind)
    elif kind == "q16":
        out = np.empty(k // 32 * 72, np.uint8)
        _check(r.ref_quantize_act16(_ptr(x), _ptr(out), k), kind)
    else:
        raise ValueError(kind)
    return out


def ref_dequantize(dtype: int, blocks: np.ndarray, k: int) -> np.ndarray:
    r = ref()
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).ravel()
    out = np.empty(k, np.float32)
    _check(r.ref_dequantize(dtype, _ptr(blocks), _ptr(out), k), "ref_dequantize")
    return out


def ref_expand_x86(dtype: int, rows: np.ndarray, k: int) -> np.ndarray:
    """The reference's x86 expansion of weight rows to fp32 (the AVX2 dequant that
    kF32ExpandGemm uses), [n, k]."""
    r = ref()
    rows = np.ascontiguousarray(np.atleast_2d(rows), dtype=np.uint8)
    out = np.empty((rows.shape[0], k), np.float32)
    for i in range(rows.shape[0]):
        _check(r.ref_expand_x86(dtype, _ptr(rows[i]), _ptr(out[i]), k), "ref_expand_x86")
    return out


def ref_expand_gemm(dtype: int, rows: np.ndarray, x: np.ndarray) -> np.ndarray:
    """The reference's kF32ExpandGemm on one thread: y [m, n] = x [m, k] . expand(rows)^T
    in its panel / gemm_panel order."""
    r = ref()
    rows = np.ascontiguousarray(np.atleast_2d(rows), dtype=np.uint8)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    m, k = x.shape
    y = np.empty((m, rows.shape[0]), np.float32)
    _check(r.ref_expand_gemm(dtype, _ptr(rows), rows.shape[1], rows.shape[0], _ptr(x), m, k, _ptr(y)),
           "ref_expand_gemm")
    return y


def ref_dot_rows(kind: int, dtype: int, w_row: np.ndarray, acts: np.ndarray, k: int) -> np.ndarray:
    """kind 0 generic per-32, 1 AVX2 per-32, 2 AVX2 super-block, 3 AVX2 sub-scaled; acts [m<=4, bytes]."""
    r = ref()
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8).ravel()
    acts = np.ascontiguousarray(np.atleast_2d(acts), dtype=np.uint8)
    m = acts.shape[0]
    out = np.empty(m, np.float32)
    rc = r.ref_dot_rows(kind, dtype, _ptr(w_row), _ptr(acts), acts.shape[1], m, k, _ptr(out))
    _check(rc, "ref_dot_rows")
    return out


def ref_split_act16(a: np.ndarray) -> np.ndarray:
    """The reference's split_act16 of int16 blocks: d, sum, hi int8[32], lo uint8[32] per 72 B."""
    r = ref()
    a = np.ascontiguousarray(a, dtype=np.uint8).ravel()
    out = np.empty_like(a)
    _check(r.ref_split_act16(_ptr(a), _ptr(out), a.size // 72), "ref_split_act16")
    return out


def ref_dot_rows16(dtype: int, w_row: np.ndarray, acts: np.ndarray, k: int) -> np.ndarray:
    """The reference's AVX2 int16 row dots (dot_rows16_*); acts [m<=4, k/32*72 bytes]."""
    r = ref()
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8).ravel()
    acts = np.ascontiguousarray(np.atleast_2d(acts), dtype=np.uint8)
    m = acts.shape[0]
    out = np.empty(m, np.float32)
    _check(r.ref_dot_rows16(dtype, _ptr(w_row), _ptr(acts), acts.shape[1], m, k, _ptr(out)), "ref_dot_rows16")
    return out


def ref_vec_dot(tier: int, dtype: int, w_row: np.ndarray, x: np.ndarray, k: int) -> float:
    """The reference's fp32-activation vec_dot (tier 0 generic, 1 AVX2) of one row."""
    r = ref()
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8).ravel()
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(1, np.float32)
    _check(r.ref_vec_dot(tier, dtype, _ptr(w_row), _ptr(x), k, _ptr(out)), "ref_vec_dot")
    return float(out[0])


def _qmm_out(m: int, k: int, mode: int, paired: bool):
    m_pad = (m + 1) // 2 * 2 if paired else m
    hi = np.zeros(m_pad * k, np.int8)
    lo = np.zeros(m_pad * k, np.uint8) if mode == 1 else None
    d = np.zeros(m_pad * (k // 32), np.float32)
    c = np.zeros(m_pad * (k // 32), np.float32)
    return hi, lo, d, c


def qmm_quantize(x: np.ndarray, mode: int, paired: bool):
    """qmm's activation buffer for the rows of x (dynacore/cpu/qmm/qmm_reference.cpp:25-51,
    440-488): (hi, lo or None, d, c) as flat arrays in the row or pair layout."""
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    hi, lo, d, c = _qmm_out(m, k, mode, paired)
    _check(lib().dqo_qmm_quantize(_ptr(x), k, m, k, mode, int(paired), _ptr(hi), _ptr(lo) if lo is not None else None,
                                  _ptr(d), _ptr(c)), "qmm_quantize")
    return hi, lo, d, c


def ref_qmm_quantize(x: np.ndarray, mode: int, paired: bool):
    """The same buffer from the reference's own ActBuffer and reference tier (oracle/_ref)."""
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    hi, lo, d, c = _qmm_out(m, k, mode, paired)
    _check(ref().ref_qmm_quantize(_ptr(x), k, m, k, mode, int(paired), _ptr(hi), _ptr(lo) if lo is not None else None,
                                  _ptr(d), _ptr(c)), "ref_qmm_quantize")
    return hi, lo, d, c


def ref_qmm_gemv(dtype: int, w_rows: np.ndarray, x: np.ndarray, mode: int, paired: bool) -> np.ndarray:
    """qmm's reference-tier gemv on x quantized into an ActBuffer (oracle/_ref): m x n fp32."""
    x = np.ascontiguousarray(x, np.float32)
    w_rows = np.ascontiguousarray(w_rows)
    m, k = x.shape
    n = w_rows.shape[0]
    y = np.zeros((m, n), np.float32)
    _check(ref().ref_qmm_gemv(dtype, _ptr(w_rows), w_rows.shape[1], n, _ptr(x), m, k, mode, int(paired), _ptr(y)),
           "ref_qmm_gemv")
    return y
