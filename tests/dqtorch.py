"""Test conveniences: torch tensors in and out of the C ABI's ctypes wrappers.

PyTorch supplies device buffers and the current HIP stream; every computation
runs in libdynaq.so's kernels.
"""
from __future__ import annotations

import torch

import dynalm_amd as dq


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def quantize(fmt: int, x: torch.Tensor) -> torch.Tensor:
    """x: [m, k] fp32 on the GPU -> [m, act_row_bytes] uint8."""
    assert x.dtype == torch.float32 and x.is_cuda and x.dim() == 2 and x.stride(1) == 1
    m, k = x.shape
    out = torch.empty((m, dq.act_row_bytes(fmt, k)), dtype=torch.uint8, device=x.device)
    dq.act_quantize(fmt, x, m, k, x.stride(0), out, stream())
    return out


def gemv(w: dq.Weight, fmt: int, acts: torch.Tensor, n0: int = 0, n1: int | None = None,
         bias: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    m = acts.shape[0]
    n1 = w.n if n1 is None else n1
    y = torch.zeros((m, w.n), dtype=torch.float32, device=acts.device) if out is None else out
    dq.gemv(w, fmt, acts, m, n0, n1, y, y.stride(0), bias, stream())
    return y


def gemm(w: dq.Weight, fmt: int, acts: torch.Tensor, n0: int = 0, n1: int | None = None,
         bias: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    m = acts.shape[0]
    n1 = w.n if n1 is None else n1
    y = torch.zeros((m, w.n), dtype=torch.float32, device=acts.device) if out is None else out
    dq.gemm(w, fmt, acts, m, n0, n1, y, y.stride(0), bias, stream())
    return y


def matmul(w: dq.Weight, x: torch.Tensor, bias: torch.Tensor | None = None,
           out: torch.Tensor | None = None) -> torch.Tensor:
    m = x.shape[0]
    y = torch.empty((m, w.n), dtype=torch.float32, device=x.device) if out is None else out
    dq.matmul(w, x, m, x.stride(0), y, y.stride(0), bias, stream())
    return y


def matmul_act(w: dq.Weight, fmt: int, x: torch.Tensor, bias: torch.Tensor | None = None,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """x . w^T under activation contract fmt (one quantize launch, then the GEMV / GEMM)."""
    m = x.shape[0]
    y = torch.empty((m, w.n), dtype=torch.float32, device=x.device) if out is None else out
    dq.matmul_act(w, fmt, x, m, x.stride(0), y, y.stride(0), bias, stream())
    return y


def partials(w: dq.Weight, fmt: int, acts: torch.Tensor):
    m = acts.shape[0]
    nu, ns = dq.partials_count(w.dtype, fmt, w.k)
    units = torch.zeros((m, w.n, nu), dtype=torch.int32, device=acts.device)
    sb = torch.zeros((m, w.n, max(ns, 1)), dtype=torch.int32, device=acts.device)
    dq.debug_partials(w, fmt, acts, m, units, sb if ns else None, stream())
    return units, sb[:, :, :ns]


def matmul_many(jobs) -> list[torch.Tensor]:
    """jobs: sequence of (w, x[, bias]) with x [m, k] fp32 on the GPU; returns the y of each
    (one dq_matmul_many call: a shared x is quantized once, decode-sized K-quant jobs of
    one k run in grouped launches)."""
    outs, spec = [], []
    for job in jobs:
        w, x = job[0], job[1]
        bias = job[2] if len(job) > 2 else None
        y = torch.empty((x.shape[0], w.n), dtype=torch.float32, device=x.device)
        outs.append(y)
        spec.append((w, x, x.shape[0], x.stride(0), y, y.stride(0), bias))
    dq.matmul_many(spec, stream())
    return outs


def act_mul(act: int, gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """act(gate) * up for [m, n] fp32 tensors on the GPU (Device::act_mul)."""
    m, n = gate.shape
    o = torch.empty((m, n), dtype=torch.float32, device=gate.device) if out is None else out
    dq.act_mul(act, gate, gate.stride(0), up, up.stride(0), m, n, o, o.stride(0), stream())
    return o


def matmul_gated(act: int, x: torch.Tensor, w_gate: dq.Weight, w_up: dq.Weight, out: torch.Tensor | None = None,
                 scratch: tuple[torch.Tensor, torch.Tensor] | None = None) -> torch.Tensor:
    """act(x . w_gate^T) * (x . w_up^T) for x [m, k] fp32 on the GPU (Device::matmul_gated)."""
    m = x.shape[0]
    o = torch.empty((m, w_gate.n), dtype=torch.float32, device=x.device) if out is None else out
    gs, us = scratch if scratch is not None else (None, None)
    dq.matmul_gated(act, x, m, x.stride(0), w_gate, w_up, o, o.stride(0), gs, us,
                    gs.stride(0) if gs is not None else 0, stream())
    return o
