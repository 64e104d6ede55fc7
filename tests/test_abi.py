"""The C-ABI library: loads, exports every symbol include/dynaq.h declares, and
validates arguments before touching a GPU (CPU only; no compute calls)."""
from __future__ import annotations

import ctypes as C
import os
import re

import pytest

import dynalm_amd as dq

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dynaq.h")


def declared_symbols() -> list[str]:
    text = open(HEADER).read()
    return re.findall(r"DQ_API\s+[\w\s\*]+?\b(dq_\w+)\s*\(", text)


def test_library_exports_every_declared_symbol():
    names = declared_symbols()
    assert len(names) >= 16
    lib = dq.lib()
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(dq.EXPORTS), set(names) ^ set(dq.EXPORTS)


def test_exports_are_the_only_public_symbols():
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", dq.lib_path()], capture_output=True, text=True).stdout
    public = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert {s for s in public if s.startswith("dq_")} == set(declared_symbols())


def test_ceiling_probe_library_is_separate():
    """bench.py's ceiling probes live in their own library: it loads and exports its
    entry points and rejects bad launches on the host; libdynaq exports none of them."""
    import subprocess

    path = os.path.join(ROOT, "dynalm_amd", "lib", "libdqceil.so")
    if not os.path.exists(path):
        pytest.skip("libdqceil.so not built")
    lib = C.CDLL(path)
    lib.dqc_read_q4k.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    lib.dqc_mfma_rate.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.POINTER(C.c_double), C.c_void_p]
    assert lib.dqc_read_q4k(None, None, 224, 16, 16, None, None) == 1
    assert lib.dqc_read_q4k(1, 1, 224, 16, 3, 1, None) == 1  # waves must divide the blocks
    assert lib.dqc_mfma_rate(256, 10, 3, 1, C.byref(C.c_double()), None) == 1  # unknown MFMA kind
    lib.dqc_read_flat.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    assert lib.dqc_read_flat(None, 1 << 20, 224, 16, 1, None) == 1
    assert lib.dqc_read_flat(1, 1000, 224, 16, 1, None) == 1  # whole KB only
    assert lib.dqc_read_flat(1, 1 << 20, 224, 17, 1, None) == 1  # at most 16 waves
    out = subprocess.run(["nm", "-D", "--defined-only", dq.lib_path()], capture_output=True, text=True).stdout
    assert "dqc_" not in out


def test_sizes():
    # dtype_row_bytes (dynacore/src/tensor/dtype.cpp:24-54)
    assert dq.row_bytes(dq.Q4_K, 4096) == 16 * 144
    assert dq.row_bytes(dq.Q6_K, 14336) == 56 * 210
    assert dq.row_bytes(dq.Q8_0, 4096) == 128 * 34
    assert dq.row_bytes(dq.Q4_0, 4096) == 128 * 18
    assert dq.row_bytes(dq.Q4_K, 100) == -1
    assert dq.row_bytes(99, 256) == -1
    assert dq.act_row_bytes(dq.ACT_Q8_K, 4096) == 16 * 292
    assert dq.act_row_bytes(dq.ACT_PER32, 4096) == 128 * 40
    assert dq.act_row_bytes(dq.ACT_Q8_0, 96) == 3 * 34
    assert dq.act_row_bytes(dq.ACT_Q8_K, 96) == -1
    assert dq.act_format_for(dq.Q4_K) == dq.ACT_Q8_K
    assert dq.act_format_for(dq.Q6_K) == dq.ACT_Q8_K
    assert dq.act_format_for(dq.Q8_0) == dq.ACT_PER32
    assert dq.act_format_for(dq.Q4_0) == dq.ACT_PER32
    assert dq.partials_count(dq.Q4_K, dq.ACT_Q8_K, 4096) == (128, 32)
    assert dq.partials_count(dq.Q6_K, dq.ACT_Q8_K, 4096) == (256, 32)
    assert dq.partials_count(dq.Q8_0, dq.ACT_PER32, 4096) == (128, 0)
    # int16 activations: ActBlockQ16 (dynacore/include/dynacore/cpu/cpu_kernels.h:77-82)
    assert dq.act_row_bytes(dq.ACT_Q16, 4096) == 128 * 72
    assert dq.act_row_bytes(dq.ACT_Q16, 96) == 3 * 72
    assert dq.partials_count(dq.Q4_K, dq.ACT_Q16, 4096) == (128, 0)
    assert dq.partials_count(dq.Q6_K, dq.ACT_Q16, 4096) == (256, 0)
    assert dq.partials_count(dq.Q8_0, dq.ACT_Q16, 4096) == (128, 0)
    # Q4_0: qmm's int16 mode runs every format (qmm_reference.cpp:68-93)
    assert dq.partials_count(dq.Q4_0, dq.ACT_Q16, 4096) == (128, 0)
    # fp32 activations (the kF32 contract): the rows themselves, no integer partials
    assert dq.act_row_bytes(dq.ACT_F32, 4096) == 4096 * 4
    assert dq.act_row_bytes(dq.ACT_F32, 100) == -1
    with pytest.raises(dq.DqError) as e:
        dq.partials_count(dq.Q4_K, dq.ACT_F32, 256)
    assert e.value.status == "unsupported"


def _upload_status(dtype, n, k, row_bytes):
    h = C.c_void_p()
    buf = (C.c_uint8 * 64)()
    return dq.lib().dq_weight_upload(dtype, C.addressof(buf), n, k, row_bytes, None, C.byref(h))


def test_invalid_arguments_rejected_before_any_gpu_call():
    """validate_matmul_shape's rules (dynacore/src/kernel/matmul_registry.cpp:264-278)
    as status codes (dynacore StatusCode values)."""
    assert _upload_status(3, 8, 256, 144) == 6            # kUnsupported weight type (i8)
    assert _upload_status(dq.Q4_K, 8, 100, 144) == 1      # k not a multiple of the block
    assert _upload_status(dq.Q4_K, 0, 256, 144) == 1      # n must be positive
    assert _upload_status(dq.Q4_K, 8, 256, 100) == 1      # row stride < row bytes
    assert b"row_bytes" in dq.lib().dq_last_error()
    assert dq.lib().dq_act_quantize(7, None, 1, 256, 256, None, None) == 6
    assert dq.lib().dq_act_quantize(dq.ACT_Q8_K, None, 1, 100, 100, None, None) == 1
    assert dq.lib().dq_gemv(None, dq.ACT_Q8_K, None, 1, 0, 1, None, 1, None, None) == 1
    assert dq.lib().dq_partials_count(dq.Q8_0, dq.ACT_Q8_K, 256, None, None) == 6
    with pytest.raises(dq.DqError) as e:
        dq.partials_count(dq.Q4_0, dq.ACT_Q8_K, 256)
    assert e.value.status == "unsupported"


def test_version():
    assert b"gfx950" in dq.lib().dq_version()


def test_matmul_many_validation_without_gpu():
    """dq_matmul_many rejects a bad call with StatusCode values before any GPU work."""
    lib = dq.lib()
    assert lib.dq_matmul_many(None, 0, None) == 0
    assert lib.dq_matmul_many(None, 1, None) == 1
    assert lib.dq_matmul_many(None, -1, None) == 1
    jobs = (dq.MatmulJob * 2)()
    assert lib.dq_matmul_many(C.cast(jobs, C.c_void_p), 2, None) == 1
    assert b"null weight" in lib.dq_last_error()
    assert C.sizeof(dq.MatmulJob) == 56


def test_gated_validation_without_gpu():
    """dq_act_mul / dq_matmul_gated reject bad arguments with StatusCode values before any GPU work."""
    lib = dq.lib()
    assert lib.dq_act_mul(dq.SILU, None, 0, None, 0, 0, 8, None, 0, None) == 0   # empty: nothing to do
    assert lib.dq_act_mul(3, None, 0, None, 0, 1, 8, None, 0, None) == 1
    assert b"activation" in lib.dq_last_error()
    assert lib.dq_act_mul(dq.GELU, None, 0, None, 0, 2, 8, None, 0, None) == 1
    assert lib.dq_act_mul(dq.GELU, None, 0, None, 0, -1, 8, None, 0, None) == 1
    assert lib.dq_matmul_gated(7, None, 1, 0, None, None, None, 0, None, None, 0, None) == 1
    assert lib.dq_matmul_gated(dq.SILU, None, 1, 0, None, None, None, 0, None, None, 0, None) == 1
    assert b"null weight" in lib.dq_last_error()


def test_qmm_buffer_layout_and_validation_without_gpu():
    """ActBuffer::prepare's layout (qmm_reference.cpp:440-454): codes, low bytes (int16), d and
    c, each rounded up to 64 bytes, pairs padded to an even row count; bad shapes, buffers and
    row ranges are rejected before any GPU call."""
    import ctypes as C

    # + the rows as per-32 (40 B) / int16 (72 B) blocks per 32 values, rounded to 64
    assert dq.qmm_act_bytes(dq.QMM_INT8, 3, 64, False) == 192 + 2 * 64 + 256
    assert dq.qmm_act_bytes(dq.QMM_INT8, 3, 64, True) == 256 + 2 * 64 + 256
    assert dq.qmm_act_bytes(dq.QMM_INT16, 2, 4096, True) == 2 * 8192 + 2 * 1024 + 2 * 128 * 72
    for bad in [(2, 1, 32, 0), (0, 1, 48, 0), (0, -1, 32, 0), (0, 1, 0, 0)]:
        assert dq.lib().dq_qmm_act_bytes(*bad) == -1
    a = dq.qmm_act_prepare(1 << 20, dq.qmm_act_bytes(dq.QMM_INT16, 4, 256, True), dq.QMM_INT16, 4, 256, True)
    assert (a.hi, a.lo, a.d, a.c, a.blocks) == (1 << 20, (1 << 20) + 1024, (1 << 20) + 2048, (1 << 20) + 2048 + 128,
                                                (1 << 20) + 2048 + 256)
    with pytest.raises(dq.DqError):
        dq.qmm_act_prepare((1 << 20) + 32, 1 << 16, dq.QMM_INT8, 4, 256, False)  # misaligned
    with pytest.raises(dq.DqError):
        dq.qmm_act_prepare(1 << 20, 100, dq.QMM_INT8, 4, 256, False)  # too small
    with pytest.raises(dq.DqError):
        dq.qmm_quantize_rows(1 << 24, 256, 2, 5, a)  # rows past m
    with pytest.raises(dq.DqError):
        dq.qmm_quantize_rows(1 << 24, 128, 0, 2, a)  # x_stride < k
    with pytest.raises(dq.DqError):
        dq.qmm_quantize_rows(1 << 24, 256, 0, 2, dq.QmmActs())  # not prepared
    assert dq.lib().dq_qmm_quantize_rows(None, 256, 1, 1, C.byref(a), None) == 0  # empty range: no launch
