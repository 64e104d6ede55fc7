"""The GPU Device shim (dynalm_amd/integration/dynaq_gpu_device.cpp): dynacore's Device
interface (dynacore/include/dynacore/device/device.h:70-219) on libdynaq, driven through the
reference's own Tensor, Storage and Status, from which oracle/_ref/libdqdevice_ref.so is
built (oracle/Makefile target `device`, harness oracle/dq_device_harness.cpp).

The harness uploads host weight tensors with Device::upload, copies x into device memory
from Device::allocate, sets a KernelPlan, runs one Device op and downloads y. Every result
is compared bit for bit with the library's own entry point for the same call: dq_matmul
under the all-integer plan, dq_matmul_plan under KernelPlan's defaults, dq_matmul_many,
dq_matmul_gated and act_mul of the two projections. An op outside the matmul path
reports kUnsupported through take_error (device.h:130-133)."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import activations, gguf_weights
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SO = os.path.join(ROOT, "oracle", "_ref", "libdqdevice_ref.so")
ALL_INT8 = dq.Plan(2, 1 << 30, 0, 1, 1 << 30, 0, 0)  # dq_matmul's plan: super-block / per-32 at every m
MATMUL, MANY, GATED, FILL = 0, 1, 2, 3
PLAN_DEFAULTS, PLAN_ALL_INT8 = 0, 1

_lib = None


def harness():
    global _lib
    if _lib is None:
        if not os.path.exists(SO):
            pytest.skip("oracle/_ref/libdqdevice_ref.so is not built (it needs the reference's sources)")
        dq.lib()  # libdynaq first: the harness links the same in-tree library
        _lib = C.CDLL(SO)
        _lib.dqdev_run.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64,
                                   C.c_int64, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p,
                                   C.c_char_p, C.c_int]
        _lib.dqdev_run.restype = C.c_int
    return _lib


def run(op, plan_kind, t, w1, w2, n, k, x, bias=None, x_stride=None):
    """One Device op through the harness; returns (y, [weight_bytes, buffer_bytes, free_bytes])."""
    m = x.shape[0]
    xs = x_stride or k
    xp = np.zeros((m, xs), np.float32)
    xp[:, :k] = x
    y = np.full(((2 if op == MANY else 1) * m, n), np.nan, np.float32)
    mem = np.zeros(3, np.int64)
    err = C.create_string_buffer(512)
    w1 = np.ascontiguousarray(w1)
    w2 = None if w2 is None else np.ascontiguousarray(w2)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = harness().dqdev_run(0, op, plan_kind, t, w1.ctypes.data, None if w2 is None else w2.ctypes.data, n, k,
                             dq.row_bytes(t, k), xp.ctypes.data, m, xs, None if b is None else b.ctypes.data,
                             y.ctypes.data, mem.ctypes.data, err, 512)
    assert rc == 0, f"status {rc}: {err.value.decode()}"
    return y, mem


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def library_matmul(w, x, n, plan_kind, bias=None):
    """The library's own call for Device::matmul under the plan."""
    m, k = x.shape
    xd = dev(x)
    y = torch.empty((m, n), device="cuda")
    b = None if bias is None else dev(bias)
    plan = ALL_INT8 if plan_kind == PLAN_ALL_INT8 else dq.plan_defaults()
    dq.matmul_plan(w, plan, xd, m, k, y, n, b, torch.cuda.current_stream().cuda_stream)
    return host(y)


KINDS = [(O.Q4_K, 1024), (O.Q6_K, 1024), (O.Q8_0, 512), (O.Q4_0, 512)]


@pytest.mark.parametrize("plan_kind", [PLAN_ALL_INT8, PLAN_DEFAULTS], ids=["all_int8", "defaults"])
@pytest.mark.parametrize("m", [1, 5, 40])
@pytest.mark.parametrize("t,k", KINDS, ids=[f"{O.TYPE_NAMES[t]}-k{k}" for t, k in KINDS])
def test_device_matmul(cuda, t, k, m, plan_kind):
    """Device::upload + Device::matmul (device.h:89,161) with a bias: the bits of dq_matmul
    (all-integer plan) or dq_matmul_plan (KernelPlan's defaults); the all-integer results
    of the K-quants also equal the oracle's."""
    n = 200
    rows = gguf_weights(t, n, k, 4000 + t + m)
    x = activations(m, k, 4001 + m)
    bias = O.normal(4002, n)
    y, mem = run(MATMUL, plan_kind, t, rows, None, n, k, x, bias=bias)
    w = dq.Weight.upload(t, rows, k)
    want = library_matmul(w, x, n, plan_kind, bias)
    assert np.array_equal(bits(y), bits(want))
    if plan_kind == PLAN_ALL_INT8 and t in (O.Q4_K, O.Q6_K):
        ref = O.matmul(t, O.ACT_Q8_K, rows, O.quantize_act(O.ACT_Q8_K, x), k, bias)
        assert np.array_equal(bits(y), bits(ref))
    assert mem[0] > 0 and mem[1] >= 4 * m * k and mem[2] > 0


def test_device_matmul_strided_rows(cuda):
    """x rows further apart than k floats (a view into a wider activation buffer)."""
    t, n, k, m = O.Q4_K, 136, 768, 6
    rows = gguf_weights(t, n, k, 4100)
    x = activations(m, k, 4101)
    y, _ = run(MATMUL, PLAN_ALL_INT8, t, rows, None, n, k, x, x_stride=k + 40)
    want = library_matmul(dq.Weight.upload(t, rows, k), x, n, PLAN_ALL_INT8)
    assert np.array_equal(bits(y), bits(want))


@pytest.mark.parametrize("plan_kind", [PLAN_ALL_INT8, PLAN_DEFAULTS], ids=["all_int8", "defaults"])
@pytest.mark.parametrize("t,m", [(O.Q4_K, 4), (O.Q6_K, 16), (O.Q4_K, 40), (O.Q8_0, 3)],
                         ids=["q4_K-m4", "q6_K-m16", "q4_K-m40", "q8_0-m3"])
def test_device_matmul_many(cuda, t, m, plan_kind):
    """Device::matmul_many (device.h:165-171) over two weights sharing x: each job's y
    has the bits of Device::matmul on it (the grouped launch where the plan selects the
    class dq_matmul runs, the per-call route otherwise)."""
    k = 512 if t == O.Q8_0 else 1024
    n = 150
    r1, r2 = gguf_weights(t, n, k, 4200 + m), gguf_weights(t, n, k, 4201 + m)
    x = activations(m, k, 4202)
    bias = O.normal(4203, n)
    y, _ = run(MANY, plan_kind, t, r1, r2, n, k, x, bias=bias)
    want1 = library_matmul(dq.Weight.upload(t, r1, k), x, n, plan_kind, bias)
    want2 = library_matmul(dq.Weight.upload(t, r2, k), x, n, plan_kind)
    assert np.array_equal(bits(y[:m]), bits(want1))
    assert np.array_equal(bits(y[m:]), bits(want2))


@pytest.mark.parametrize("plan_kind", [PLAN_ALL_INT8, PLAN_DEFAULTS], ids=["all_int8", "defaults"])
@pytest.mark.parametrize("t,m", [(O.Q4_K, 1), (O.Q4_K, 16), (O.Q6_K, 7), (O.Q4_K, 40)],
                         ids=["q4_K-m1", "q4_K-m16", "q6_K-m7", "q4_K-m40"])
def test_device_matmul_gated(cuda, t, m, plan_kind):
    """Device::matmul_gated (device.h:188-199), SiLU: under the all-integer plan the
    bits of dq_matmul_gated (one fused launch for decode rows), under the defaults those
    of act_mul over the two projections as Device::matmul computes them."""
    import dqtorch as T

    k, n = 1024, 130
    rg, ru = gguf_weights(t, n, k, 4300 + m), gguf_weights(t, n, k, 4301 + m)
    x = activations(m, k, 4302)
    y, _ = run(GATED, plan_kind, t, rg, ru, n, k, x)
    wg, wu = dq.Weight.upload(t, rg, k), dq.Weight.upload(t, ru, k)
    if plan_kind == PLAN_ALL_INT8:
        want = host(T.matmul_gated(O.SILU, dev(x), wg, wu))
    else:
        g = dev(library_matmul(wg, x, n, plan_kind))
        u = dev(library_matmul(wu, x, n, plan_kind))
        want = host(T.act_mul(O.SILU, g, u))
    assert np.array_equal(bits(y), bits(want))


def test_device_op_outside_the_path_reports_unsupported(cuda):
    """Device::fill is outside the quantized-matmul path: take_error() returns kUnsupported
    (the harness returns 0 only then)."""
    t, n, k = O.Q4_K, 64, 256
    run(FILL, PLAN_DEFAULTS, t, gguf_weights(t, n, k, 4400), None, n, k, activations(2, k, 4401))
