"""Kernel selection (accuracy classes) without a GPU: dq_select against the reference's
own select_matmul (dynacore/src/kernel/matmul_registry.cpp:287-429), compiled from its
sources into oracle/_ref and recorded in tests/golden/select_matmul.npz by
tests/golden/make_select_golden.py, over a grid of shapes and KernelPlans; the plan
defaults and the FFN-down plan as known answers (kernel_plan.h:34-148,
dynalm/src/model/transformer.cpp:541-550)."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import pytest

import dynalm_amd as dq
from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "select_matmul.npz")
# MatmulActFormat (matmul_registry.h:141) -> dq_act_format
ACT_OF = {0: dq.ACT_F32, 1: dq.ACT_PER32, 2: dq.ACT_Q8_K, 3: dq.ACT_SX, 4: dq.ACT_Q16}


def plan_of(row) -> dq.Plan:
    return dq.Plan(*[int(v) for v in row[:6]], int(row[6]) & 0xFFFFFFFF, int(row[7]), int(row[8]))


def test_defaults_are_kernel_plan_defaults():
    # KernelPlan's member initializers (kernel_plan.h:34,58,66,77,81,92,148,156,158)
    assert dq.plan_defaults().as_dict() == {
        "expand_min_rows": 2, "int8_decode_max_rows": 4, "int16_decode_max_rows": 0,
        "int8_superblock_min_rows": 0, "int8_superblock_max_rows": 8, "int8_subscale_min_rows": 1,
        "matmul_disabled": 0, "qmm": 1, "qmm_gemm_min_rows": 9}


def test_ffn_down_plan():
    # transformer.cpp:541-550: int16 up to max(int8 rows, super-block max rows), no int8
    d = dq.plan_ffn_down()
    assert (d.int8_decode_max_rows, d.int16_decode_max_rows) == (0, 8)
    neon = dq.plan_defaults()
    neon.int8_decode_max_rows = 64
    assert (dq.plan_ffn_down(neon).int8_decode_max_rows, dq.plan_ffn_down(neon).int16_decode_max_rows) == (0, 64)
    off = dq.plan_defaults()
    off.int8_decode_max_rows = 0  # --int8-decode 0 keeps fp32 everywhere (no int16 either)
    assert dq.plan_ffn_down(off).int16_decode_max_rows == 0


def _no_qmm() -> dq.Plan:
    p = dq.plan_defaults()
    p.qmm = 0
    return p


def test_default_classes_known_answers():
    """The accuracy classes a default-plan engine gets (kernel_plan.h:50-101,149-158):
    with qmm (this GPU has its kernels), qmm's gemv on per-32 rows up to the int8 row
    limit; past it the int8 family's sub-scaled rows (K-quants, to 8 rows) and then fp32.
    Without qmm, the x86 tiers' classes."""
    for t in (dq.Q4_K, dq.Q6_K, dq.Q8_0, dq.Q4_0):
        for m in range(1, 5):
            s = dq.select(m, 4096, 4096, t)
            assert (s.kernel, s.act) == (dq.KERNEL_QMM_GEMV, dq.ACT_PER32), (t, m)
    for t in (dq.Q4_K, dq.Q6_K):
        for m in range(5, 9):
            assert (dq.select(m, 4096, 4096, t).kernel, dq.select(m, 4096, 4096, t).act) == (
                dq.KERNEL_INT8_SUBSCALED, dq.ACT_SX)
        for m in range(1, 9):
            s = dq.select(m, 4096, 4096, t, _no_qmm())
            assert (s.kernel, s.act) == (dq.KERNEL_INT8_SUBSCALED, dq.ACT_SX), (t, m)
        assert dq.select(9, 4096, 4096, t).kernel == dq.KERNEL_F32_EXPAND_GEMM
        assert dq.select(512, 4096, 4096, t).act == dq.ACT_F32
    for t in (dq.Q8_0, dq.Q4_0):
        for m in range(1, 5):
            s = dq.select(m, 4096, 4096, t, _no_qmm())
            assert (s.kernel, s.act) == (dq.KERNEL_INT8_PER32, dq.ACT_PER32)
        assert dq.select(5, 4096, 4096, t).kernel == dq.KERNEL_F32_EXPAND_GEMM
        assert dq.select(5, 4096, 4096, t, x_dense=False).kernel == dq.KERNEL_F32_ROW_DOT
    # the engine's plan on a qmm-accelerated backend (engine.cpp:365-375): qmm at any size
    eng = dq.plan_defaults()
    eng.int8_decode_max_rows = 1 << 30
    for t in (dq.Q4_K, dq.Q8_0, dq.Q4_0, dq.Q6_K):
        assert (dq.select(512, 14336, 4096, t, eng).kernel, dq.select(512, 14336, 4096, t, eng).act) == (
            dq.KERNEL_QMM_GEMM, dq.ACT_PER32)
        assert dq.select(8, 14336, 4096, t, eng).kernel == dq.KERNEL_QMM_GEMV
    # and its FFN down plan (transformer.cpp:541-550): int16 rows through qmm at any size
    eng_down = dq.plan_ffn_down(eng)
    assert (dq.select(512, 4096, 14336, dq.Q6_K, eng_down).kernel, dq.select(512, 4096, 14336, dq.Q6_K, eng_down).act) == (
        dq.KERNEL_QMM_GEMM, dq.ACT_Q16)
    down = dq.plan_ffn_down()
    for t in (dq.Q6_K, dq.Q4_K, dq.Q8_0, dq.Q4_0):
        assert (dq.select(8, 4096, 14336, t, down).kernel, dq.select(8, 4096, 14336, t, down).act) == (
            dq.KERNEL_QMM_GEMV, dq.ACT_Q16)
        assert dq.select(9, 4096, 14336, t, down).act == dq.ACT_F32
        nq = dq.plan_ffn_down(_no_qmm())
        assert (dq.select(8, 4096, 14336, t, nq).kernel, dq.select(8, 4096, 14336, t, nq).act) == (
            dq.KERNEL_INT16_ROWS, dq.ACT_Q16)


def test_select_matches_reference_table():
    g = np.load(GOLDEN)
    plans = [plan_of(p) for p in g["plans"]]
    bad = []
    for (pi, t, m, n, k, dense), kid, act in zip(g["cases"], g["kernel"], g["act"]):
        s = dq.select(int(m), int(n), int(k), int(t), plans[int(pi)], bool(dense))
        if (s.kernel, s.act) != (int(kid), ACT_OF[int(act)]):
            bad.append((int(pi), int(t), int(m), int(k), int(dense), (s.kernel, s.act), (int(kid), int(act))))
    assert not bad, f"{len(bad)} of {len(g['kernel'])} differ, e.g. {bad[:5]}"
    assert set(np.unique(g["kernel"])) == {1, 2, 7, 8, 9, 13, 14, 15}


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs the reference sources)")
def test_select_matches_reference_live():
    """Random plans and shapes against the reference's select_matmul itself."""
    r = O.ref()
    rng = np.random.default_rng(7)
    for _ in range(4000):
        p = [int(rng.integers(1, 5)), int(rng.choice([0, 1, 4, 8, 64, 1 << 30])), int(rng.choice([0, 4, 8, 16])),
             int(rng.choice([0, 1, 3, 9])), int(rng.choice([0, 4, 8, 16, 1 << 30])), int(rng.choice([0, 1, 2, 5])),
             int(rng.integers(0, 1 << 16)), int(rng.integers(0, 2)), int(rng.choice([1, 4, 9, 33]))]
        t = int(rng.choice([6, 10, 14, 16]))
        k = int(rng.choice([32, 96, 256, 512, 4096, 14336]))
        if t in (14, 16) and k % 256:
            k = 256
        m = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 64, 100, 512]))
        dense = int(rng.integers(0, 2))
        a = C.c_int(-1)
        kid = r.ref_select_matmul(m, 4096, k, t, dense, *p[:6], C.c_uint32(p[6]), p[7], p[8], C.byref(a))
        s = dq.select(m, 4096, k, t, dq.Plan(*p), bool(dense))
        assert (s.kernel, s.act) == (kid, ACT_OF[a.value]), (p, t, m, k, dense)


def test_select_rejects_bad_shapes():
    with pytest.raises(dq.DqError) as e:
        dq.select(0, 64, 256, dq.Q4_K)
    assert e.value.status == "invalid_argument"
    with pytest.raises(dq.DqError) as e:
        dq.select(1, 64, 100, dq.Q4_K)
    assert e.value.status == "invalid_argument"
    with pytest.raises(dq.DqError) as e:
        dq.select(1, 64, 256, 3)
    assert e.value.status == "unsupported"
