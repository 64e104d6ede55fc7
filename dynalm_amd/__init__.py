"""dynalm_amd -- MI355X-native block-quantized matmul (Python mirror of the C ABI).

The product is the C-ABI library ``dynalm_amd/lib/libdynaq.so`` (include/dynaq.h):
hand-written gfx950 HIP kernels behind dynacore's quantized-matmul entry points.
This module binds it with ctypes; device buffers are passed as integer device
pointers and streams as integer hipStream_t handles, so any allocator (PyTorch
included) can supply them. Loading fails loudly when the library is missing:
there is no CPU fallback.

Entry points mirror the reference's operator interface (names and argument
meaning of dynacore/include/dynacore/cpu/qmm.h:116-137 and
dynacore/include/dynacore/device/device.h:89-161):

    Weight.upload(dtype, rows, k)      Device::upload + prepack_weight
    act_quantize(fmt, x, m, k, ...)    qmm::Kernels::quantize_row / QuantizeActFn
    gemv(w, fmt, acts, m, n0, n1, ...) qmm::Kernels::gemv / DotQ8RowsNFn
    gemm(w, fmt, acts, m, n0, n1, ...) qmm::Kernels::gemm
    matmul(w, x, m, ...)               Device::matmul
    matmul_many(jobs)                  Device::matmul_many
    act_mul(act, gate, up, ...)        Device::act_mul
    matmul_gated(act, x, wg, wu, ...)  Device::matmul_gated
    GgufFile.open(path)                dynalm's GgufFile::open / open_parts (host mmap + parse)
    GgufFile.upload(name)              Device::upload of a GGUF tensor

Errors raise DqError carrying dynacore's StatusCode value
(dynacore/include/dynacore/base/status.h:19-32).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

__all__ = [
    "Q4_0", "Q8_0", "Q4_K", "Q6_K", "ACT_PER32", "ACT_Q8_0", "ACT_Q8_K", "ACT_SX", "ACT_Q16", "ACT_F32", "GEMV_MAX_ROWS", "matmul_act",
    "DqError", "lib", "lib_path", "row_bytes", "act_row_bytes", "act_format_for", "Weight",
    "act_quantize", "gemv", "gemm", "matmul", "matmul_many", "MatmulJob", "partials_count", "debug_partials",
    "SILU", "GELU", "GELU_TANH", "act_mul", "matmul_gated", "GgufFile", "GgufTensor", "EXPORTS",
    "MatmulShape", "External", "matmul_noalloc", "NOALLOC_SCRATCH_BYTES", "Plan", "Selection",
    "plan_defaults", "plan_ffn_down", "select", "matmul_plan", "KERNEL_NAMES", "KERNEL_QMM_GEMM", "KERNEL_QMM_GEMV",
]

Q4_0, Q8_0, Q4_K, Q6_K = 6, 10, 14, 16
ACT_PER32, ACT_Q8_0, ACT_Q8_K, ACT_SX, ACT_Q16, ACT_F32 = 0, 1, 2, 3, 4, 5
GEMV_MAX_ROWS = 16
SILU, GELU, GELU_TANH = 0, 1, 2  # dq_activation (dynacore Activation, device/ops.h:14)

STATUS_NAMES = {
    0: "ok", 1: "invalid_argument", 2: "not_found", 3: "already_exists", 4: "out_of_memory",
    5: "resource_exhausted", 6: "unsupported", 7: "io_error", 8: "corrupt", 9: "cancelled",
    10: "deadline_exceeded", 11: "internal",
}

_HERE = os.path.dirname(os.path.abspath(__file__))


def lib_path() -> str:
    return os.environ.get("DYNAQ_LIB", os.path.join(_HERE, "lib", "libdynaq.so"))


_P = C.c_void_p
_I64 = C.c_int64
_I = C.c_int

# Every symbol include/dynaq.h declares, with its ctypes signature.
class QmmActs(C.Structure):
    """dq_qmm_acts: qmm::Acts (dynacore/include/dynacore/cpu/qmm.h:71-79), device pointers."""
    _fields_ = [("mode", C.c_int32), ("paired", C.c_int32), ("m", C.c_int64), ("k", C.c_int64),
                ("hi", C.c_void_p), ("lo", C.c_void_p), ("d", C.c_void_p), ("c", C.c_void_p),
                ("blocks", C.c_void_p)]


QMM_INT8, QMM_INT16 = 0, 1  # dq_qmm_mode (qmm::ActMode)

EXPORTS = {
    "dq_version": (C.c_char_p, []),
    "dq_last_error": (C.c_char_p, []),
    "dq_row_bytes": (_I64, [_I, _I64]),
    "dq_act_row_bytes": (_I64, [_I, _I64]),
    "dq_act_format_for": (_I, [_I]),
    "dq_weight_upload": (_I, [_I, _P, _I64, _I64, _I64, _P, C.POINTER(_P)]),
    "dq_weight_upload_device": (_I, [_I, _P, _I64, _I64, _I64, _P, C.POINTER(_P)]),
    "dq_weight_download": (_I, [_P, _P, _I64, _P]),
    "dq_weight_free": (_I, [_P]),
    "dq_weight_info": (_I, [_P, C.POINTER(_I), C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_I64)]),
    "dq_act_quantize": (_I, [_I, _P, _I64, _I64, _I64, _P, _P]),
    "dq_qmm_act_bytes": (_I64, [_I, _I64, _I64, _I]),
    "dq_qmm_act_prepare": (_I, [_P, _I64, _I, _I64, _I64, _I, C.POINTER(QmmActs), _P]),
    "dq_qmm_quantize_rows": (_I, [_P, _I64, _I64, _I64, C.POINTER(QmmActs), _P]),
    "dq_qmm_gemv": (_I, [_P, _I64, _I64, C.POINTER(QmmActs), _I64, _I, _P, _I64, _P, _P]),
    "dq_qmm_gemm": (_I, [_P, _I64, _I64, C.POINTER(QmmActs), _P, _I64, _P, _P]),
    "dq_gemv": (_I, [_P, _I, _P, _I64, _I64, _I64, _P, _I64, _P, _P]),
    "dq_gemm": (_I, [_P, _I, _P, _I64, _I64, _I64, _P, _I64, _P, _P]),
    "dq_matmul": (_I, [_P, _P, _I64, _I64, _P, _I64, _P, _P]),
    "dq_matmul_noalloc": (_I, [_P, _P, _I64, _I64, _P, _I64, _P, _P]),
    "dq_matmul_many": (_I, [_P, _I64, _P]),
    "dq_matmul_act": (_I, [_P, _I, _P, _I64, _I64, _P, _I64, _P, _P]),
    "dq_act_mul": (_I, [_I, _P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P]),
    "dq_gguf_open": (_I, [C.c_char_p, C.POINTER(_P)]),
    "dq_gguf_close": (_I, [_P]),
    "dq_gguf_info": (_I, [_P, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.POINTER(_I64), C.POINTER(_I64)]),
    "dq_gguf_find_tensor": (_I64, [_P, C.c_char_p]),
    "dq_gguf_tensor_info": (_I, [_P, _I64, _P]),
    "dq_gguf_get_uint": (_I, [_P, C.c_char_p, C.POINTER(C.c_uint64)]),
    "dq_gguf_get_string": (_I, [_P, C.c_char_p, C.POINTER(C.c_char_p), C.POINTER(_I64)]),
    "dq_gguf_upload_weight": (_I, [_P, _I64, _P, C.POINTER(_P)]),
    "dq_matmul_gated": (_I, [_I, _P, _I64, _I64, _P, _P, _P, _I64, _P, _P, _I64, _P]),
    "dq_partials_count": (_I, [_I, _I, _I64, C.POINTER(_I64), C.POINTER(_I64)]),
    "dq_debug_partials": (_I, [_P, _I, _P, _I64, _P, _P, _P]),
    "dq_external_create": (_I, [_I, _I64, _I64, C.POINTER(_P)]),
    "dq_external_free": (_I, [_P]),
    "dq_external_eligible": (_I, [_P, _P, _P]),
    "dq_external_run": (_I, [_P, _P, _I64, _I64, _P, _I, _I64, _I64, _I64, _P, _P, _I64]),
    "dq_external_forget": (_I, [_P, _P]),
    "dq_external_get_stats": (_I, [_P, _P]),
    "dq_external_set_plan": (_I, [_P, _P]),
    "dq_plan_defaults": (_I, [_P]),
    "dq_plan_ffn_down": (_I, [_P, _P]),
    "dq_select": (_I, [_P, _P, _P]),
    "dq_matmul_plan": (_I, [_P, _P, _P, _I64, _I64, _P, _I64, _P, _P]),
}


class DqError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {message}")
        self.code = code
        self.status = STATUS_NAMES.get(code, str(code))


_lib = None


def lib() -> C.CDLL:
    """The loaded C-ABI library (raises if it is not built)."""
    global _lib
    if _lib is None:
        path = lib_path()
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built: run `python -m dynalm_amd.build` (no CPU fallback exists)")
        L = C.CDLL(path)
        for name, (res, args) in EXPORTS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise DqError(rc, lib().dq_last_error().decode(errors="replace"))


def _ptr(x) -> int | None:
    """Device pointer of a torch tensor / int / None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    raise TypeError(f"expected a device pointer, got {type(x)!r}")


def row_bytes(dtype: int, k: int) -> int:
    return int(lib().dq_row_bytes(dtype, k))


def act_row_bytes(fmt: int, k: int) -> int:
    return int(lib().dq_act_row_bytes(fmt, k))


def act_format_for(dtype: int) -> int:
    return int(lib().dq_act_format_for(dtype))


class Weight:
    """A weight matrix in the device layout (owns its device memory)."""

    def __init__(self, handle: int):
        self._h = C.c_void_p(handle)
        dt, n, k, nbytes = _I(), _I64(), _I64(), _I64()
        _check(lib().dq_weight_info(self._h, C.byref(dt), C.byref(n), C.byref(k), C.byref(nbytes)))
        self.dtype, self.n, self.k, self.device_bytes = dt.value, n.value, k.value, nbytes.value

    @classmethod
    def upload(cls, dtype: int, rows: np.ndarray, k: int, stream: int = 0) -> "Weight":
        """Upload GGUF rows (uint8 [n, row_bytes]) from host memory."""
        rows = np.ascontiguousarray(np.atleast_2d(rows), dtype=np.uint8)
        h = C.c_void_p()
        _check(lib().dq_weight_upload(dtype, rows.ctypes.data, rows.shape[0], k, rows.shape[1], stream, C.byref(h)))
        return cls(h.value)

    @classmethod
    def upload_device(cls, dtype: int, dev_rows, n: int, k: int, row_stride: int, stream: int = 0) -> "Weight":
        h = C.c_void_p()
        _check(lib().dq_weight_upload_device(dtype, _ptr(dev_rows), n, k, row_stride, stream, C.byref(h)))
        return cls(h.value)

    def download(self, stream: int = 0) -> np.ndarray:
        rb = row_bytes(self.dtype, self.k)
        out = np.zeros((self.n, rb), np.uint8)
        _check(lib().dq_weight_download(self._h, out.ctypes.data, rb, stream))
        return out

    @property
    def handle(self) -> C.c_void_p:
        if self._h is None:
            raise ValueError("weight was freed")
        return self._h

    def free(self) -> None:
        if getattr(self, "_h", None) is not None and _lib is not None:
            lib().dq_weight_free(self._h)
        self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def act_quantize(fmt: int, x, m: int, k: int, x_stride: int, out, stream: int = 0) -> None:
    _check(lib().dq_act_quantize(fmt, _ptr(x), m, k, x_stride, _ptr(out), stream))


def qmm_act_bytes(mode: int, m: int, k: int, paired: bool) -> int:
    """Bytes of qmm's activation buffer for the shape (ActBuffer::prepare's layout)."""
    n = lib().dq_qmm_act_bytes(mode, m, k, int(paired))
    if n < 0:
        raise DqError(3, f"qmm acts: mode {mode}, m {m}, k {k}")
    return n


def qmm_act_prepare(base, nbytes: int, mode: int, m: int, k: int, paired: bool, stream: int = 0) -> QmmActs:
    """ActBuffer::prepare (qmm_reference.cpp:440-469) on a device buffer of nbytes."""
    a = QmmActs()
    _check(lib().dq_qmm_act_prepare(_ptr(base), nbytes, mode, m, k, int(paired), C.byref(a), stream))
    return a


def qmm_quantize_rows(x, x_stride: int, r0: int, r1: int, acts: QmmActs, stream: int = 0) -> None:
    """ActBuffer::quantize_rows (qmm_reference.cpp:472-488): rows [r0, r1) of x."""
    _check(lib().dq_qmm_quantize_rows(_ptr(x), x_stride, r0, r1, C.byref(acts), stream))


def qmm_gemv(w: Weight, n0: int, n1: int, acts: QmmActs, r0: int, rows: int, y, y_stride: int, bias=None,
             stream: int = 0) -> None:
    """qmm::Kernels::gemv on a qmm activation buffer (rows [r0, r0 + rows))."""
    _check(lib().dq_qmm_gemv(w.handle, n0, n1, C.byref(acts), r0, rows, _ptr(y), y_stride, _ptr(bias), stream))


def qmm_gemm(w: Weight, n0: int, n1: int, acts: QmmActs, y, y_stride: int, bias=None, stream: int = 0) -> None:
    """qmm::Kernels::gemm on a qmm activation buffer (every row)."""
    _check(lib().dq_qmm_gemm(w.handle, n0, n1, C.byref(acts), _ptr(y), y_stride, _ptr(bias), stream))


def gemv(w: Weight, fmt: int, acts, m: int, n0: int, n1: int, y, y_stride: int, bias=None, stream: int = 0) -> None:
    _check(lib().dq_gemv(w.handle, fmt, _ptr(acts), m, n0, n1, _ptr(y), y_stride, _ptr(bias), stream))


def gemm(w: Weight, fmt: int, acts, m: int, n0: int, n1: int, y, y_stride: int, bias=None, stream: int = 0) -> None:
    _check(lib().dq_gemm(w.handle, fmt, _ptr(acts), m, n0, n1, _ptr(y), y_stride, _ptr(bias), stream))


def matmul(w: Weight, x, m: int, x_stride: int, y, y_stride: int, bias=None, stream: int = 0) -> None:
    _check(lib().dq_matmul(w.handle, _ptr(x), m, x_stride, _ptr(y), y_stride, _ptr(bias), stream))


NOALLOC_SCRATCH_BYTES = 16 << 20  # DQ_NOALLOC_SCRATCH_BYTES


def matmul_noalloc(w: Weight, x, m: int, x_stride: int, y, y_stride: int, bias=None, stream: int = 0) -> None:
    """dq_matmul with its temporaries in the library's static device array (no allocation)."""
    _check(lib().dq_matmul_noalloc(w.handle, _ptr(x), m, x_stride, _ptr(y), y_stride, _ptr(bias), stream))


def matmul_act(w: Weight, fmt: int, x, m: int, x_stride: int, y, y_stride: int, bias=None, stream: int = 0) -> None:
    """y = x . w^T (+ bias) under activation contract fmt (ACT_SX: dynacore's sub-scaled int8)."""
    _check(lib().dq_matmul_act(w.handle, fmt, _ptr(x), m, x_stride, _ptr(y), y_stride, _ptr(bias), stream))


class MatmulJob(C.Structure):
    """dq_matmul_job (include/dynaq.h): one matmul of matmul_many."""
    _fields_ = [("w", _P), ("x", _P), ("m", _I64), ("x_stride", _I64), ("y", _P), ("y_stride", _I64),
                ("bias", _P)]


def matmul_many(jobs, stream: int = 0) -> None:
    """jobs: sequence of (w, x, m, x_stride, y, y_stride, bias) tuples (Device::matmul_many)."""
    arr = (MatmulJob * max(len(jobs), 1))()
    for i, (w, x, m, xs, y, ys, bias) in enumerate(jobs):
        arr[i] = MatmulJob(w.handle.value if isinstance(w, Weight) else w, _ptr(x), m, xs, _ptr(y), ys, _ptr(bias))
    _check(lib().dq_matmul_many(C.cast(arr, _P), len(jobs), stream))


def act_mul(act: int, gate, gate_stride: int, up, up_stride: int, m: int, n: int, out, out_stride: int,
            stream: int = 0) -> None:
    """out = act(gate) * up elementwise (Device::act_mul)."""
    _check(lib().dq_act_mul(act, _ptr(gate), gate_stride, _ptr(up), up_stride, m, n, _ptr(out), out_stride, stream))


def matmul_gated(act: int, x, m: int, x_stride: int, w_gate: Weight, w_up: Weight, out, out_stride: int,
                 gate_scratch=None, up_scratch=None, scratch_stride: int = 0, stream: int = 0) -> None:
    """out = act(x . w_gate^T) * (x . w_up^T) (Device::matmul_gated); scratch optional."""
    _check(lib().dq_matmul_gated(act, _ptr(x), m, x_stride, w_gate.handle, w_up.handle, _ptr(out), out_stride,
                                 _ptr(gate_scratch), _ptr(up_scratch), scratch_stride, stream))


def partials_count(dtype: int, fmt: int, k: int) -> tuple[int, int]:
    u, s = _I64(), _I64()
    _check(lib().dq_partials_count(dtype, fmt, k, C.byref(u), C.byref(s)))
    return int(u.value), int(s.value)


def debug_partials(w: Weight, fmt: int, acts, m: int, units, sb=None, stream: int = 0) -> None:
    _check(lib().dq_debug_partials(w.handle, fmt, _ptr(acts), m, _ptr(units), _ptr(sb), stream))


# ------------------------------------------------------------------ GGUF files


class GgufTensor(C.Structure):
    """dq_gguf_tensor (include/dynaq.h): one entry of the tensor directory."""
    _fields_ = [("name", C.c_char_p), ("ggml_type", C.c_uint32), ("dtype", C.c_int32), ("n_dims", C.c_int32),
                ("dims", _I64 * 4), ("offset", C.c_uint64), ("nbytes", C.c_uint64), ("part", C.c_int32),
                ("data", _P)]

    @property
    def shape(self) -> tuple[int, ...]:
        return tuple(int(self.dims[d]) for d in range(self.n_dims))


class GgufFile:
    """A GGUF model mapped read-only (all parts of a split model): dynalm's GgufFile
    (dynalm/src/loader/gguf/gguf.h:77-125) over the library's parser."""

    def __init__(self, handle: int):
        self._h = C.c_void_p(handle)

    @classmethod
    def open(cls, path: str) -> "GgufFile":
        h = _P()
        _check(lib().dq_gguf_open(os.fsencode(path), C.byref(h)))
        return cls(h.value)

    def close(self) -> None:
        if self._h:
            lib().dq_gguf_close(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self) -> dict:
        v, a, n, p = C.c_uint32(), C.c_uint64(), _I64(), _I64()
        _check(lib().dq_gguf_info(self._h, C.byref(v), C.byref(a), C.byref(n), C.byref(p)))
        return {"version": v.value, "alignment": a.value, "n_tensors": n.value, "n_parts": p.value}

    def tensor(self, i: int) -> GgufTensor:
        t = GgufTensor()
        _check(lib().dq_gguf_tensor_info(self._h, i, C.byref(t)))
        return t

    def tensors(self) -> list[GgufTensor]:
        return [self.tensor(i) for i in range(self.info()["n_tensors"])]

    def find(self, name: str) -> int:
        return int(lib().dq_gguf_find_tensor(self._h, name.encode()))

    def get_uint(self, key: str) -> int:
        v = C.c_uint64()
        _check(lib().dq_gguf_get_uint(self._h, key.encode(), C.byref(v)))
        return v.value

    def get_string(self, key: str) -> str:
        p, n = C.c_char_p(), _I64()
        _check(lib().dq_gguf_get_string(self._h, key.encode(), C.byref(p), C.byref(n)))
        return C.string_at(p, n.value).decode()

    def data(self, name: str) -> bytes:
        """The tensor's bytes as they lie in the file."""
        i = self.find(name)
        if i < 0:
            raise DqError(2, f"tensor {name!r} not found")
        t = self.tensor(i)
        return C.string_at(t.data, t.nbytes)

    def upload(self, name: str, stream: int = 0) -> "Weight":
        i = self.find(name)
        if i < 0:
            raise DqError(2, f"tensor {name!r} not found")
        h = _P()
        _check(lib().dq_gguf_upload_weight(self._h, i, stream, C.byref(h)))
        return Weight(h.value)


class MatmulShape(C.Structure):
    """dq_matmul_shape (dynacore MatmulShape, kernel/matmul_registry.h:87-91)."""
    _fields_ = [("m", _I64), ("n", _I64), ("k", _I64), ("dtype", C.c_int32), ("x_dense", C.c_int32)]


# dq_kernel: dynacore MatmulKernelId values (kernel/matmul_registry.h:33-51)
KERNEL_QMM_GEMM, KERNEL_QMM_GEMV = 1, 2
KERNEL_INT8_SUBSCALED, KERNEL_INT8_SUPERBLOCK, KERNEL_INT8_PER32 = 7, 8, 9
KERNEL_INT16_ROWS, KERNEL_F32_EXPAND_GEMM, KERNEL_F32_ROW_DOT = 13, 14, 15
F32_GEMM_MIN_ROWS = 16  # DQ_F32_GEMM_MIN_ROWS: the expand class on the matrix cores from here on
KERNEL_NAMES = {1: "qmm_gemm", 2: "qmm_gemv", 7: "int8_subscaled", 8: "int8_superblock", 9: "int8_per32",
                13: "int16_rows", 14: "f32_expand_gemm", 15: "f32_row_dot"}


class Plan(C.Structure):
    """dq_plan: KernelPlan's matmul knobs (kernel/kernel_plan.h:34-148)."""
    _fields_ = [("expand_min_rows", C.c_int32), ("int8_decode_max_rows", C.c_int32),
                ("int16_decode_max_rows", C.c_int32), ("int8_superblock_min_rows", C.c_int32),
                ("int8_superblock_max_rows", C.c_int32), ("int8_subscale_min_rows", C.c_int32),
                ("matmul_disabled", C.c_uint32), ("qmm", C.c_int32), ("qmm_gemm_min_rows", C.c_int32)]

    def as_dict(self) -> dict:
        return {f: getattr(self, f) for f, _ in self._fields_}


class Selection(C.Structure):
    """dq_selection: the kernel (dq_kernel) and the activation format it quantizes x to."""
    _fields_ = [("kernel", C.c_int32), ("act", C.c_int32)]


def plan_defaults() -> Plan:
    """KernelPlan::defaults() without environment overrides."""
    p = Plan()
    _check(lib().dq_plan_defaults(C.byref(p)))
    return p


def plan_ffn_down(base: Plan | None = None) -> Plan:
    """The FFN down projection's plan derived from base (transformer.cpp:541-550)."""
    p = Plan()
    _check(lib().dq_plan_ffn_down(C.byref(base) if base is not None else None, C.byref(p)))
    return p


def select(m: int, n: int, k: int, dtype: int, plan: Plan | None = None, x_dense: bool = True) -> Selection:
    """select_matmul over this library's kernels (no GPU needed)."""
    out = Selection()
    shape = MatmulShape(m, n, k, dtype, int(x_dense))
    _check(lib().dq_select(C.byref(shape), C.byref(plan) if plan is not None else None, C.byref(out)))
    return out


def matmul_plan(w: Weight, plan: Plan | None, x, m: int, x_stride: int, y, y_stride: int, bias=None,
                stream: int = 0) -> None:
    """Device::matmul under a KernelPlan (None: the defaults)."""
    _check(lib().dq_matmul_plan(w.handle, C.byref(plan) if plan is not None else None, _ptr(x), m, x_stride, _ptr(y),
                                y_stride, _ptr(bias), stream))


class ExternalStats(C.Structure):
    _fields_ = [("runs", _I64), ("uploads", _I64), ("hits", _I64), ("evictions", _I64), ("resident_bytes", _I64),
                ("resident_weights", _I64)]


def external_eligible(shape: MatmulShape, weight: int, adapter: "External | None" = None) -> bool:
    """dq_external_eligible: a pure shape rule (no GPU needed with adapter None)."""
    h = adapter._h if adapter is not None else None
    return bool(lib().dq_external_eligible(h, C.byref(shape), weight))


class External:
    """dq_external: matmuls on host (numpy) arrays, with device copies of the weights
    kept across calls (the ExternalMatmulKernel shape of dynacore's CpuDevice)."""

    def __init__(self, device: int = 0, min_rows: int = 1, max_resident_bytes: int = 0):
        h = _P()
        _check(lib().dq_external_create(device, min_rows, max_resident_bytes, C.byref(h)))
        self._h = h

    def close(self) -> None:
        if self._h:
            _check(lib().dq_external_free(self._h))
            self._h = _P()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def eligible(self, m: int, n: int, k: int, dtype: int, weight: int, x_dense: bool = True) -> bool:
        return external_eligible(MatmulShape(m, n, k, dtype, int(x_dense)), weight, self)

    def run(self, x, w_rows, dtype: int, k: int, bias=None, y=None):
        """x: [m, k] float32 (row stride from the array), w_rows: [n, row_bytes] uint8
        GGUF rows; returns y [m, n] float32 (or fills the given y)."""
        import numpy as np

        assert x.dtype == np.float32 and x.ndim == 2 and x.strides[1] == 4
        assert w_rows.dtype == np.uint8 and w_rows.ndim == 2 and w_rows.strides[1] == 1
        m, n = x.shape[0], w_rows.shape[0]
        if y is None:
            y = np.empty((m, n), np.float32)
        assert y.dtype == np.float32 and y.strides[1] == 4
        b = None
        if bias is not None:
            bias = np.ascontiguousarray(bias, np.float32)
            b = bias.ctypes.data
        _check(lib().dq_external_run(self._h, x.ctypes.data, m, x.strides[0] // 4, w_rows.ctypes.data, dtype, n, k,
                                     w_rows.strides[0], b, y.ctypes.data, y.strides[0] // 4))
        return y

    def set_plan(self, plan: Plan | None) -> None:
        """Device::set_kernel_plan for the adapter (None: the defaults)."""
        _check(lib().dq_external_set_plan(self._h, C.byref(plan) if plan is not None else None))

    def forget(self, w_rows) -> None:
        _check(lib().dq_external_forget(self._h, w_rows.ctypes.data))

    def stats(self) -> dict:
        st = ExternalStats()
        _check(lib().dq_external_get_stats(self._h, C.byref(st)))
        return {f: getattr(st, f) for f, _ in ExternalStats._fields_}
