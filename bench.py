"""Benchmark of the block-quantized matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Headline (BASELINE.json metric "Q4_K GEMV HBM GB/s (% peak) at M=1; Q4_K GEMM int8
TOPS (% peak) at M=512"): one step = dq_matmul on one fp32 activation row: Q8_K
quantization (inside the GEMV kernel) + the Q4_K GEMV at config 3's gate/up shape
(K=4096, N=14336, M=1), one kernel launch per step, weights resident
in HBM and rotated over copies totalling well over the 256 MB Infinity Cache (as
dynalm/benchmarks/bench_decode_matmul.cpp:11-14 rotates layers). `value` is the
step's algorithmic bytes (packed weights + quantized activations + fp32 output) per
second. A second leg times the config 4 prefill GEMM (M=512) in int8 TOPS.

Both `roofline` objects use per-kernel durations from HIP events around one replay
of a HIP graph that holds exactly K back-to-back launches of that kernel alone (the
Python launch loop costs ~5 us per call, close to the kernel itself; its timing is
reported beside). `cpu_baseline` times the
call dynacore makes on x86 for this step (Q4_K x sub-scaled int8: quantize_act_sx and
dot_q8_sx_rows_n on its ThreadPool, dynacore/cpu/cpu_device.cpp:941-960,
dynacore/src/kernel/matmul_registry.cpp:139-165) compiled from the reference sources
(oracle/_ref) on the host's physical cores, on a bounded sample.
Inputs are synthetic: random valid Q4_K blocks (fp16 d, dmin in U(0.002, 0.02)) and
N(0, 1) activations; timing does not depend on the values.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K GEMV HBM GB/s (% peak) at M=1; Q4_K GEMM int8 TOPS (% peak) at M=512"
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E
PEAK_INT8_TOPS = 5000.0   # MI355X dense int8 MFMA
PEAK_F16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 MFMA
K, N = 4096, 14336        # config 3 gate/up, config 4
Q4K_ROW = K // 256 * 144
Q8K_ROW = K // 256 * 292


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def random_q4k_rows(n: int, k: int, seed: int) -> np.ndarray:
    """Random valid Q4_K blocks: random scales/codes, fp16 d and dmin in U(0.002, 0.02)."""
    rng = np.random.default_rng(seed)
    rows = rng.integers(0, 256, (n, k // 256, 144), dtype=np.uint8)
    dd = rng.uniform(0.002, 0.02, (n, k // 256, 2)).astype(np.float16)
    rows[:, :, 0:4] = dd.view(np.uint8).reshape(n, k // 256, 4)
    return rows.reshape(n, -1)


def time_launches(fn, iters: int, warmup: int) -> float:
    """Average ms per call of fn(i, stream) over `iters` back-to-back calls issued from
    Python on the current stream (HIP events on that stream)."""
    import torch

    stream = torch.cuda.current_stream().cuda_stream
    for i in range(warmup):
        fn(i, stream)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(iters):
        fn(i, stream)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def time_graph(fn, iters: int, warmup: int) -> float:
    """Average ms per call of fn(i, stream) over exactly `iters` calls replayed from one
    HIP graph. The calls are warmed up eagerly first (so that no library scratch is
    allocated during capture), then captured on a side stream; the timed region is one
    replay, bracketed by HIP events on the stream that launches it. This removes the
    Python / ctypes launch cost (a few us per call) from the GPU timeline."""
    import torch

    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        for i in range(warmup):
            fn(i, side.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for i in range(iters):
            fn(i, side.cuda_stream)
    g.replay()  # untimed: first replay uploads the graph
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / iters
    del g
    return ms


def host_cpu() -> dict:
    """The host CPU as bench.py reports it: model, ISA flags of interest, cores."""
    info = {"cpu": "unknown", "isa": []}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and info["cpu"] == "unknown":
                    info["cpu"] = line.split(":", 1)[1].strip()
                elif line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    info["isa"] = [f for f in ("avx2", "fma", "f16c", "avx_vnni", "avx512f", "avx512_vnni", "amx_int8")
                                   if f in flags]
                    break
    except OSError:
        pass
    return info


def llc_of_cpus(cpus) -> tuple[int, int]:
    """(bytes of one last-level cache, number of distinct last-level caches) over the
    given CPUs, from sysfs (the highest cache index that is not an instruction cache)."""
    base = "/sys/devices/system/cpu"
    size, seen = 0, set()
    for c in sorted(cpus):
        d = f"{base}/cpu{c}/cache"
        try:
            idx = sorted(int(e[5:]) for e in os.listdir(d) if e.startswith("index"))
        except OSError:
            continue
        for i in reversed(idx):
            try:
                with open(f"{d}/index{i}/type") as f:
                    if f.read().strip() == "Instruction":
                        continue
                with open(f"{d}/index{i}/size") as f:
                    txt = f.read().strip()
                with open(f"{d}/index{i}/shared_cpu_list") as f:
                    shared = f.read().strip()
            except OSError:
                continue
            mult = {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}.get(txt[-1:], 1)
            size = max(size, int(txt.rstrip("KMG")) * mult)
            seen.add(shared)
            break
    return size, len(seen)


def cpu_baseline(w_host: np.ndarray, budget_s: float) -> dict:
    """dynacore's x86 decode call for this step, timed on the host cores: the
    reference's own CpuDevice decode path for the sub-scaled int8 class (its x86
    default for M=1, quantize_act_sx included in every call) on its own ThreadPool,
    created once, over the weight rows with its grain (oracle/_ref, ref_bench_decode_sx)."""
    from oracle import oracle as O

    x = O.normal(7, K)
    nbytes = Q4K_ROW * N + K // 256 * 320 + 4 * N
    host = host_cpu()
    r = O.ref()
    if r is not None and r.ref_has_avx2():
        import ctypes as C

        phys, logical = r.ref_physical_cores(), r.ref_logical_cores()
        try:
            cpus = os.sched_getaffinity(0)
        except AttributeError:
            cpus = set(range(os.cpu_count() or 1))
        share = len(cpus)
        threads = max(1, min(phys, share, 16))  # the GPU box's CPU share is 16
        llc, n_llc = llc_of_cpus(cpus)
        if llc == 0:
            llc, n_llc = int(r.ref_llc_bytes()), 1
        # rotate over copies totalling at least twice all the last-level caches the threads can use
        copies = int(min(16, max(2, -(-2 * max(llc * n_llc, 1) // w_host.nbytes) + 1)))
        ws = [w_host] + [w_host.copy() for _ in range(copies - 1)]
        ptrs = (C.c_void_p * copies)(*[w.ctypes.data for w in ws])
        y = np.empty(N, np.float32)
        chunks = 32  # KernelPlan::matmul_chunks_per_thread (kernel_plan.h:40)

        def run(th: int, iters: int) -> float:
            ns = r.ref_bench_decode_sx(O.Q4_K, ptrs, copies, Q4K_ROW, N, x.ctypes.data, 1, K, y.ctypes.data, th,
                                       chunks, iters)
            assert ns > 0, f"ref_bench_decode_sx: {ns}"
            return ns / iters / 1e9

        per = run(threads, 2)
        iters = max(4, int(budget_s / max(per, 1e-6)))
        sec = run(threads, iters)
        sec1 = run(1, 1)
        iters1 = max(2, int(0.25 * budget_s / max(sec1, 1e-6)))
        sec1 = run(1, iters1)
        return {"value": round(nbytes / sec / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "reference",
                "ms_per_call": round(sec * 1e3, 4), "tokens_per_s": round(1.0 / sec, 1),
                "one_thread": {"value": round(nbytes / sec1 / 1e9, 2), "ms_per_call": round(sec1 * 1e3, 4),
                               "calls": iters1},
                "sample": f"{iters} calls of the full K=4096 N=14336 M=1 Q4_K decode matmul as dynacore's CpuDevice "
                          f"runs it on x86 (quantize_act_sx + dot_q8_sx_rows_n, kInt8Subscaled) on its ThreadPool of "
                          f"{threads} threads (grain_for over rows, {chunks} chunks per thread), {copies} rotated "
                          f"weight copies ({copies * w_host.nbytes >> 20} MiB; {n_llc} last-level caches of "
                          f"{llc >> 20} MiB over the process's CPUs)",
                "cpu": host["cpu"], "isa": host["isa"], "physical_cores": phys, "logical_cores": logical,
                "cpu_share": share, "llc_bytes": llc, "llc_count": n_llc, "weight_copies": copies}
    # scalar oracle restatement on a bounded sample of rows, scaled to N
    a = O.quantize_act(O.ACT_SX, x[None])
    rows = 256
    t0 = time.perf_counter()
    O.matmul(O.Q4_K, O.ACT_SX, w_host[:rows], a, K)
    sec = (time.perf_counter() - t0) * N / rows
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "ms_per_call": round(sec * 1e3, 3), "tokens_per_s": round(1.0 / sec, 2),
            "sample": f"{rows} of {N} rows of the Q4_K x sub-scaled GEMV (scalar oracle), scaled to N",
            "cpu": host["cpu"], "isa": host["isa"]}


# Config 5: Qwen2.5-1.5B-shaped decode step, M = 16: per layer (name, dtype, n, k)
QWEN_LAYER = [("q", 14, 1536, 1536), ("k", 14, 256, 1536), ("v", 16, 256, 1536), ("o", 14, 1536, 1536),
              ("gate", 14, 8960, 1536), ("up", 14, 8960, 1536), ("down", 16, 1536, 8960)]
QWEN_LAYERS = 28
QWEN_LM_HEAD = ("lm_head", 16, 151936, 1536)


def random_rows(dtype: int, n: int, k: int, seed: int) -> np.ndarray:
    """Random valid K-quant blocks (fp16 d, dmin in U(0.002, 0.02))."""
    nb = k // 256
    bb = 144 if dtype == 14 else 210
    rng = np.random.default_rng(seed)
    rows = rng.integers(0, 256, (n, nb, bb), dtype=np.uint8)
    dd = rng.uniform(0.002, 0.02, (n, nb, 2)).astype(np.float16).view(np.uint8).reshape(n, nb, 4)
    if dtype == 14:
        rows[:, :, 0:4] = dd
    else:
        rows[:, :, 208:210] = dd[:, :, 0:2]
    return rows.reshape(n, -1)


def decode_stack(steps: int, stream: int) -> dict:
    """Config 5: the 28-layer matmul stack plus lm_head of one decode step at M = 16,
    in the order a transformer step issues it (dynalm/src/model/transformer.cpp:605-718):
    per layer matmul_many(q, k, v) on the attention input, o, matmul_gated(SiLU, gate,
    up) on the MLP input (the compiler's gate/up/act_mul fusion,
    dynacore/include/dynacore/ir/passes.h:79), down on its output; then lm_head. Each
    call quantizes its input to Q8_K on the GPU (in the kernel for the small ones) and
    runs the skinny MFMA GEMV. Timed as one graph replay per `steps` steps."""
    import torch

    import dynalm_amd as dq

    m = 16
    uploads = {}
    for name, t, n, k in QWEN_LAYER + [QWEN_LM_HEAD]:
        rows = random_rows(t, n, k, sum(map(ord, name)))
        src = torch.from_numpy(rows).cuda()
        count = 1 if name == "lm_head" else QWEN_LAYERS
        uploads[name] = [dq.Weight.upload_device(t, src, n, k, rows.shape[1], stream) for _ in range(count)]
        del src
    xs = {stage: torch.randn((m, k), device="cuda") for stage, k in
          (("attn", 1536), ("o", 1536), ("mlp", 1536), ("down", 8960))}
    ys = {name: torch.empty((m, n), device="cuda") for name, _, n, _ in QWEN_LAYER + [QWEN_LM_HEAD]}
    total_bytes = sum(n * (k // 256) * (144 if t == 14 else 210) * (1 if name == "lm_head" else QWEN_LAYERS)
                      for name, t, n, k in QWEN_LAYER + [QWEN_LM_HEAD])
    shapes = {name: (n, k) for name, _, n, k in QWEN_LAYER + [QWEN_LM_HEAD]}

    def job(name: str, layer: int, stage: str):
        n, k = shapes[name]
        return (uploads[name][layer], xs[stage], m, k, ys[name], n, None)

    def step(_i: int, st: int) -> None:
        for layer in range(QWEN_LAYERS):
            dq.matmul_many([job("q", layer, "attn"), job("k", layer, "attn"), job("v", layer, "attn")], st)
            dq.matmul(*job("o", layer, "o"), st)
            dq.matmul_gated(dq.SILU, xs["mlp"], m, 1536, uploads["gate"][layer], uploads["up"][layer], xs["down"],
                            8960, stream=st)
            dq.matmul(*job("down", layer, "down"), st)
        dq.matmul(*job("lm_head", 0, "o"), st)

    ms = time_graph(step, steps, 2)
    out = {"workload": "config 5: Qwen2.5-1.5B decode-step matmul stack (28 layers + lm_head), M=16; per layer "
                       "matmul_many(q,k,v), o, matmul_gated(silu, gate, up), down",
           "ms_per_step": round(ms, 4), "weight_bytes": total_bytes,
           "gbs": round(total_bytes / (ms * 1e-3) / 1e9, 1), "tokens_per_s": round(m / (ms * 1e-3), 1)}
    for ws in uploads.values():
        for w in ws:
            w.free()
    return out


def prefill_sweep(ms: list[int], weights, gen) -> list[dict]:
    """Config 4's sweep: dq_matmul on M fp32 rows (Q8_K quantization on the GPU, then
    the kernel dq_matmul dispatches to: the skinny MFMA GEMV up to 16 rows, the MFMA
    GEMM above), K=4096 N=14336, rotated weights, graph replay. Beside it the engine's
    plan (qmm on per-32 rows at any M, dq_matmul_plan): per-32 quantize + the f16 per-32
    GEMM (split K where its tiles leave CUs idle)."""
    import torch

    import dynalm_amd as dq

    out = []
    ng = min(4, len(weights))
    eng = dq.plan_defaults()
    eng.int8_decode_max_rows = 1 << 30
    for m in ms:
        x = torch.randn((m, K), generator=gen, device="cuda", dtype=torch.float32)
        y = torch.empty((m, N), dtype=torch.float32, device="cuda")
        iters = max(10, min(50, 20000 // m))
        log(f"prefill sweep M={m} x{iters}")
        ms_call = time_graph(lambda i, st: dq.matmul(weights[i % ng], x, m, K, y, N, None, st), iters, 3)
        tops = 2.0 * m * N * K / (ms_call * 1e-3) / 1e12
        cus = torch.cuda.get_device_properties(0).multi_processor_count
        f16 = m > 128 and -(-m // 128) * -(-N // 256) * 8 >= 5 * cus  # the f16 GEMM's rule (gemm_h16_pays)
        ms_eng = time_graph(lambda i, st: dq.matmul_plan(weights[i % ng], eng, x, m, K, y, N, None, st), iters, 3)
        out.append({"m": m, "kernel": "skinny MFMA GEMV" if m <= 16 else "f16 MFMA GEMM" if f16 else "int8 MFMA GEMM",
                    "ms_per_call": round(ms_call, 4), "tops": round(tops, 1),
                    "pct_peak_int8": round(100 * tops / PEAK_INT8_TOPS, 2), "tokens_per_s": round(m / (ms_call * 1e-3), 1),
                    "engine_plan_per32_ms_per_call": round(ms_eng, 4)})
        del x, y
    return out


def prefill_other_types(gen) -> list[dict]:
    """dq_matmul at M = 512 for the other weight types of a Q4_K_M / Q8_0 / Q4_0 model:
    Q6_K FFN down (K=14336 N=4096) on the Q6_K GEMM, Q8_0 4096 x 4096 and Q4_0
    K=4096 N=14336 on the 32-value block GEMM (quantization included, 2 rotated copies).
    For Q6_K also dq_matmul_act on per-32 and int16 rows (k_gemm_q6k_x)."""
    import torch

    import dynalm_amd as dq

    out = []
    m = 512
    for name, dtype, n, k in (("q6_K", dq.Q6_K, 4096, 14336), ("q8_0", dq.Q8_0, 4096, 4096),
                              ("q4_0", dq.Q4_0, 14336, 4096)):
        rb = k // 256 * 210 if dtype == dq.Q6_K else k // 32 * (34 if dtype == dq.Q8_0 else 18)
        rng = np.random.default_rng(dtype)
        ws = []
        for _ in range(2):
            rows = rng.integers(0, 256, (n, rb), dtype=np.uint8)
            if dtype == dq.Q6_K:
                rows = random_rows(16, n, k, int(rng.integers(1 << 30)))
            else:  # fp16 d in U(0.002, 0.02) at the start of each block
                bb = 34 if dtype == dq.Q8_0 else 18
                blk = rows.reshape(n, -1, bb)
                blk[:, :, 0:2] = rng.uniform(0.002, 0.02, blk.shape[:2]).astype(np.float16).view(np.uint8).reshape(
                    n, -1, 2)
            ws.append(dq.Weight.upload(dtype, rows, k))
        x = torch.randn((m, k), generator=gen, device="cuda", dtype=torch.float32)
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        log(f"prefill {name} M={m}")
        ms_call = time_graph(lambda i, st: dq.matmul(ws[i % 2], x, m, k, y, n, None, st), 20, 3)
        tops = 2.0 * m * n * k / (ms_call * 1e-3) / 1e12
        rec = {"weights": f"{name} K={k} N={n}", "m": m, "ms_per_call": round(ms_call, 4), "tops": round(tops, 1),
               "pct_peak_int8": round(100 * tops / PEAK_INT8_TOPS, 2)}
        if dtype == dq.Q6_K:
            # the engine plan's contracts for this matrix (qmm int8 rows; the FFN-down plan's
            # int16 rows): quantize + operand layout + k_gemm_q6k_x on the f16 matrix cores
            for key, fmt in (("per32", dq.ACT_PER32), ("int16", dq.ACT_Q16)):
                log(f"prefill {name} M={m} {key}")
                ms_f = time_graph(lambda i, st, fmt=fmt: dq.matmul_act(ws[i % 2], fmt, x, m, k, y, n, None, st), 20, 3)
                tf = 2.0 * m * n * k / (ms_f * 1e-3) / 1e12
                rec[f"{key}_ms_per_call"] = round(ms_f, 4)
                rec[f"{key}_tops"] = round(tf, 1)
                rec[f"{key}_pct_peak_f16"] = round(100 * tf / PEAK_F16_TFLOPS, 2)
        out.append(rec)
        del ws, x, y
    return out


COPY_BYTES = 64 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4k_gemv_m1_gemm_m512_traffic.md")


def pmc_leg(weights, x, acts, y, stream) -> None:
    """Launches for the counter passes: the copy kernel first (COPY_BYTES read and
    written, the calibration of FETCH_SIZE / WRITE_SIZE), then the measured kernels: the
    fused and plain M=1 GEMVs, the M=512 Q8_K GEMM and the M=512 default-plan prefill."""
    import torch

    import dynalm_amd as dq

    src = torch.ones(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    nc = len(weights)
    for i in range(2 * nc):
        dq.matmul(weights[i % nc], x, 1, K, y, N, None, stream)
    dq.act_quantize(dq.ACT_Q8_K, x, 1, K, K, acts, stream)
    for i in range(2 * nc):
        dq.gemv(weights[i % nc], dq.ACT_Q8_K, acts, 1, 0, N, y, N, None, stream)
    m = 512
    xg = torch.randn((m, K), device="cuda", dtype=torch.float32)
    ag = torch.empty((m, Q8K_ROW), dtype=torch.uint8, device="cuda")
    yg = torch.empty((m, N), dtype=torch.float32, device="cuda")
    dq.act_quantize(dq.ACT_Q8_K, xg, m, K, K, ag, stream)
    for i in range(4):
        dq.gemm(weights[i % nc], dq.ACT_Q8_K, ag, m, 0, N, yg, N, None, stream)
    # the default-plan prefill: per-32 quantize, k_act32_from_p32, k_gemm_q4k_p32
    eng = dq.plan_defaults()
    eng.int8_decode_max_rows = 1 << 30
    for i in range(4):
        dq.matmul_plan(weights[i % nc], eng, xg, m, K, yg, N, None, stream)
    torch.cuda.synchronize()
    log("pmc leg done")


def pmc_f16_leg(stream) -> None:
    """Launches for the counter passes of the f16 GEMMs on the per-32 and int16 contracts
    (dq_matmul_act): the copy kernel first (calibration), then three calls each of Q6_K
    K=14336 N=4096 (config 3's down projection) per-32 and int16 at M=512 and per-32 at
    M=16, and Q4_K K=4096 N=14336 int16 at M=512 and per-32 at M=16."""
    import torch

    import dynalm_amd as dq

    src = torch.ones(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    for name, t, n, k, cases in (
            ("q6_K", dq.Q6_K, 4096, 14336, ((512, "per32"), (512, "int16"), (16, "per32"))),
            ("q4_K", dq.Q4_K, 14336, 4096, ((512, "int16"), (16, "per32")))):
        rows = random_rows(t, n, k, 5)
        w = dq.Weight.upload(t, rows, k)
        for m, fname in cases:
            fmt = dq.ACT_PER32 if fname == "per32" else dq.ACT_Q16
            log(f"pmc f16 leg: {name} x {fname}, m={m}")
            x = torch.randn((m, k), device="cuda")
            y = torch.empty((m, n), device="cuda")
            for _ in range(3):
                dq.matmul_act(w, fmt, x, m, k, y, n, None, stream)
            torch.cuda.synchronize()
        w.free()
    log("pmc f16 leg done")


def ceilings(steps: int, warmup: int) -> dict:
    """The two ceilings the headline kernels are quoted against, measured here with
    libdqceil.so (dynalm_amd/csrc/dq_ceiling.hip): the decode GEMV's loads alone
    (same grid, same per-wave runs and offsets, no arithmetic) over 33 MB and over
    132 MB (four times K at the same launch shape), rotated over copies totalling
    528 MB as the GEMV is; the plain read of the same 33 MB at ten launch shapes (the
    best one is the read ceiling the GEMV's launch shape gives up against); and
    back-to-back int8 MFMAs on every SIMD."""
    import ctypes as C

    import torch

    lib = C.CDLL(os.path.join(ROOT, "dynalm_amd", "lib", "libdqceil.so"))
    lib.dqc_read_q4k.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    lib.dqc_mfma_rate.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.POINTER(C.c_double), C.c_void_p]
    groups, waves = N // 64, 16
    out = {"kernel": "dqc_read_q4k: the GEMV's nontemporal dwordx4 loads (8 KB codes + 1 KB headers per super-block "
                     "and 64 rows) and one fp32 store per row, no arithmetic",
           "launch": f"{groups} workgroups x {waves} waves (one per 64-row group, as k_gemv)"}
    for label, nblk, copies in (("33MB", K // 256, 16), ("132MB", 4 * K // 256, 4)):
        qs = [torch.full((groups * nblk * 8192,), 1, dtype=torch.uint8, device="cuda") for _ in range(copies)]
        hd = [torch.full((groups * nblk * 1024,), 1, dtype=torch.uint8, device="cuda") for _ in range(copies)]
        y = torch.empty(groups * 64, dtype=torch.float32, device="cuda")

        def read(i: int, st: int) -> None:
            rc = lib.dqc_read_q4k(qs[i % copies].data_ptr(), hd[i % copies].data_ptr(), groups, nblk, waves,
                                  y.data_ptr(), st)
            assert rc == 0, f"dqc_read_q4k: {rc}"

        ms = time_graph(read, steps, warmup)
        nbytes = groups * nblk * (8192 + 1024) + groups * 64 * 4
        out[label] = {"bytes": nbytes, "blocks_per_wave": nblk // waves, "copies": copies,
                      "ms_per_launch": round(ms, 5), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)}
        del qs, hd, y
    torch.cuda.empty_cache()
    # the plain read of the GEMV's weight bytes at ten launch shapes (16 rotated copies, as
    # the GEMV): the best one-launch read of them, the GEMV's shape first
    lib.dqc_read_flat.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    wbytes = Q4K_ROW * N
    flat = [torch.full((wbytes,), 1, dtype=torch.uint8, device="cuda") for _ in range(16)]
    sink = torch.empty(8192, dtype=torch.int32, device="cuda")
    sweep = {}
    for wgs, waves in ((N // 64, 16), (256, 16), (448, 8), (512, 8), (896, 4), (1024, 4), (1792, 2), (2048, 2),
                       (3584, 1), (4096, 1)):
        def flat_read(i: int, st: int, wgs=wgs, waves=waves) -> None:
            rc = lib.dqc_read_flat(flat[i % 16].data_ptr(), wbytes, wgs, waves, sink.data_ptr(), st)
            assert rc == 0, f"dqc_read_flat: {rc}"

        ms = time_graph(flat_read, steps, warmup)
        sweep[f"{wgs}x{waves}"] = {"ms_per_launch": round(ms, 5), "gbs": round(wbytes / (ms * 1e-3) / 1e9, 1)}
    best = max(sweep, key=lambda key: sweep[key]["gbs"])
    out["read_shape_sweep"] = {"bytes": wbytes, "kernel": "dqc_read_flat: one contiguous piece per wave, "
                               "nontemporal dwordx4, up to 8 KB in flight per wave", "shapes": sweep,
                               "best": best, "best_gbs": sweep[best]["gbs"]}
    del flat, sink
    torch.cuda.empty_cache()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    mfma = {"launch": f"{cus} workgroups x 8 waves (two per SIMD), 8 independent accumulators per wave"}
    for label, kind, iters in (("16x16x64", 0, 4000), ("32x32x32", 1, 2000), ("f16_32x32x16", 2, 2000)):
        buf = torch.empty(cus * 512, dtype=torch.int32, device="cuda")
        ops = C.c_double(0.0)

        def rate(i: int, st: int) -> None:
            rc = lib.dqc_mfma_rate(cus, iters, kind, buf.data_ptr(), C.byref(ops), st)
            assert rc == 0, f"dqc_mfma_rate: {rc}"

        ms = time_graph(rate, 5, 2)
        mfma[label] = {"ms_per_launch": round(ms, 4), "tops": round(ops.value / (ms * 1e-3) / 1e12, 1)}
    out["mfma"] = mfma
    return out


def measured_traffic() -> dict:
    """HBM bytes per launch of the measured kernels, as the committed counter summary
    records them (lines `traffic <kernel> <bytes>`); empty if it is absent."""
    out = {}
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic":
                    out[parts[1]] = int(parts[2])
    except OSError:
        pass
    return out


def output_checks(w, x, acts, xg, ag, m: int, stream: int) -> dict:
    """Bit-equality of the timed paths with independent kernels on the same inputs."""
    import torch

    import dynalm_amd as dq

    y_fused = torch.empty((1, N), device="cuda")
    y_gemv = torch.empty((1, N), device="cuda")
    dq.matmul(w, x, 1, K, y_fused, N, None, stream)
    dq.act_quantize(dq.ACT_Q8_K, x, 1, K, K, acts, stream)
    dq.gemv(w, dq.ACT_Q8_K, acts, 1, 0, N, y_gemv, N, None, stream)
    yg = torch.empty((m, N), device="cuda")
    dq.gemm(w, dq.ACT_Q8_K, ag, m, 0, N, yg, N, None, stream)
    idx = torch.linspace(0, m - 1, 16, device="cuda").round().long()
    a16 = ag[idx].contiguous()
    y16 = torch.empty((16, N), device="cuda")
    dq.gemv(w, dq.ACT_Q8_K, a16, 16, 0, N, y16, N, None, stream)
    y1 = torch.empty((1, N), device="cuda")
    dq.gemv(w, dq.ACT_Q8_K, a16[:1], 1, 0, N, y1, N, None, stream)
    torch.cuda.synchronize()
    bits = lambda t: t.view(torch.int32)
    return {"fused_step_eq_gemv": bool(torch.equal(bits(y_fused), bits(y_gemv))),
            "gemm_rows_eq_skinny_gemv": bool(torch.equal(bits(yg[idx]), bits(y16))),
            "gemm_row_eq_gemv": bool(torch.equal(bits(yg[idx[:1]]), bits(y1))),
            "rows_checked": [int(i) for i in idx.tolist()]}


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--copies", type=int, default=16, help="rotated weight copies (x 33 MB)")
    ap.add_argument("--gemm-m", type=int, default=512)
    ap.add_argument("--gemm-iters", type=int, default=50)
    ap.add_argument("--sweep", default="16,64,128,512,2048",
                    help="config 4 prefill sweep: dq_matmul (quantization + the kernel dq_matmul picks) at these M "
                         "('' to skip)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--stack-steps", type=int, default=20, help="config 5 decode-stack steps (0: skip)")
    ap.add_argument("--pmc-leg", action="store_true",
                    help="no timing: a 64 MiB copy kernel (counter calibration), then a few launches of each "
                         "measured kernel, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes")
    ap.add_argument("--pmc-f16-leg", action="store_true",
                    help="no timing: a 64 MiB copy kernel, then three calls each of the per-32 / int16 f16 GEMMs "
                         "(Q6_K down projection at M=512 and 16, Q4_K at M=512 int16 and M=16 per-32), for "
                         "rocprofv3 --pmc passes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the path would shard the weight "
              f"rows across GPUs, see DESIGN.md; no multi-GPU figure is produced)", file=sys.stderr)
        sys.exit(2)

    import torch

    import dynalm_amd as dq

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream().cuda_stream
    log(f"device {torch.cuda.get_device_name(0)}; building inputs")

    # ---- weights: `copies` device copies of one random Q4_K matrix
    w_host = random_q4k_rows(N, K, 20261201)
    w_src = torch.from_numpy(w_host).cuda()
    weights = [dq.Weight.upload_device(dq.Q4_K, w_src, N, K, Q4K_ROW, stream) for _ in range(args.copies)]
    del w_src
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)

    # ---- decode step: dq_matmul, M=1: fp32 x -> Q8_K in the kernel -> Q4_K GEMV -> fp32 y
    x = torch.randn((1, K), generator=gen, device="cuda", dtype=torch.float32)
    acts = torch.empty((1, Q8K_ROW), dtype=torch.uint8, device="cuda")
    y = torch.empty((1, N), dtype=torch.float32, device="cuda")
    nc = args.copies

    def step(i: int, st: int) -> None:
        dq.matmul(weights[i % nc], x, 1, K, y, N, None, st)

    def gemv_only(i: int, st: int) -> None:
        dq.gemv(weights[i % nc], dq.ACT_Q8_K, acts, 1, 0, N, y, N, None, st)

    if args.pmc_leg:
        pmc_leg(weights, x, acts, y, stream)
        return
    if args.pmc_f16_leg:
        pmc_f16_leg(stream)
        return

    log(f"decode step x{args.steps} (warmup {args.warmup})")
    ms_step = time_graph(step, args.steps, args.warmup)
    ms_step_eager = time_launches(step, args.steps, args.warmup)
    log("GEMV on pre-quantized activations")
    dq.act_quantize(dq.ACT_Q8_K, x, 1, K, K, acts, stream)
    ms_gemv = time_graph(gemv_only, args.steps, args.warmup)
    bytes_step = Q4K_ROW * N + Q8K_ROW + 4 * N
    value = bytes_step / (ms_step * 1e-3) / 1e9
    # the step is one kernel (k_gemv_slab<16, 2, true>: Q4_K x Q8_K, M=1): its launch time is ms_step
    achieved = value

    # ---- the gated pair at the step's shape: act(x . Wg^T) * (x . Wu^T), one launch
    pairs = [(weights[2 * j], weights[2 * j + 1]) for j in range(nc // 2)]
    yq = torch.empty((1, N), dtype=torch.float32, device="cuda")

    def gated(i: int, st: int) -> None:
        wg, wu = pairs[i % len(pairs)]
        dq.matmul_gated(dq.SILU, x, 1, K, wg, wu, y, N, stream=st)

    def two_matmuls(i: int, st: int) -> None:
        wg, wu = pairs[i % len(pairs)]
        dq.matmul(wg, x, 1, K, y, N, None, st)
        dq.matmul(wu, x, 1, K, yq, N, None, st)

    ms_gated = ms_two = None
    if pairs:
        log(f"gated pair x{args.steps // 2}")
        ms_gated = time_graph(gated, args.steps // 2, args.warmup)
        ms_two = time_graph(two_matmuls, args.steps // 2, args.warmup)

    # ---- prefill GEMM, M = 512
    m = args.gemm_m
    xg = torch.randn((m, K), generator=gen, device="cuda", dtype=torch.float32)
    ag = torch.empty((m, Q8K_ROW), dtype=torch.uint8, device="cuda")
    dq.act_quantize(dq.ACT_Q8_K, xg, m, K, K, ag, stream)
    yg = torch.empty((m, N), dtype=torch.float32, device="cuda")
    ng = min(4, nc)

    def gemm(i: int, st: int) -> None:
        dq.gemm(weights[i % ng], dq.ACT_Q8_K, ag, m, 0, N, yg, N, None, st)

    log(f"GEMM M={m} x{args.gemm_iters}")
    ms_gemm = time_graph(gemm, args.gemm_iters, 3)
    ops = 2.0 * m * N * K
    tops = ops / (ms_gemm * 1e-3) / 1e12

    # ---- the timed kernels' outputs, checked against independent kernels that compute the
    # same integers and fp32 steps (no oracle here): the fused M = 1 step against the GEMV on
    # separately quantized rows, and sampled GEMM rows against the M = 1 GEMV and the skinny
    # MFMA GEMV on those rows; every pair must agree bit for bit
    checks = output_checks(weights[0], x, acts, xg, ag, m, stream)
    log(f"output checks: {checks}")

    # ---- the fp32 expand + GEMM class at the same shape (the default plan's choice for
    # m > 8 dense fp32 rows): weights expanded in LDS, v_mfma_f32_32x32x2_f32
    yf = torch.empty((m, N), dtype=torch.float32, device="cuda")

    def f32_gemm(i: int, st: int) -> None:
        dq.matmul_plan(weights[i % ng], None, xg, m, K, yf, N, None, st)

    def f32_row_dot(i: int, st: int) -> None:
        dq.matmul_act(weights[i % ng], dq.ACT_F32, xg, m, K, yf, N, None, st)

    log(f"fp32 expand GEMM M={m}")
    ms_f32 = time_graph(f32_gemm, 10, 2)
    ms_f32_rows = time_graph(f32_row_dot, 3, 1)
    tf32 = ops / (ms_f32 * 1e-3) / 1e12

    # ---- the default plans: KernelPlan::defaults() with this GPU's qmm caps. Prefill under
    # the engine's plan on a backend with accelerated qmm (int8 rows unbounded,
    # dynalm/src/runtime/engine.cpp:365-375): qmm's gemm on per-32 rows (per-32 quantize,
    # f16 operand layout, k_gemm_q4k_p32). Decode (M = 1) under the defaults: qmm's gemv on
    # per-32 rows; and without qmm, the x86 tiers' sub-scaled class (the CPU baseline's).
    eng = dq.plan_defaults()
    eng.int8_decode_max_rows = 1 << 30
    noqmm = dq.plan_defaults()
    noqmm.qmm = 0
    sel_pre = dq.select(m, N, K, dq.Q4_K, eng)
    sel_dec, sel_x86 = dq.select(1, N, K, dq.Q4_K), dq.select(1, N, K, dq.Q4_K, noqmm)

    def prefill_plan(i: int, st: int) -> None:
        dq.matmul_plan(weights[i % ng], eng, xg, m, K, yf, N, None, st)

    def decode_plan(plan):
        return lambda i, st: dq.matmul_plan(weights[i % nc], plan, x, 1, K, y, N, None, st)

    log(f"default plans: prefill M={m} ({dq.KERNEL_NAMES[sel_pre.kernel]}), decode M=1 "
        f"({dq.KERNEL_NAMES[sel_dec.kernel]}; without qmm {dq.KERNEL_NAMES[sel_x86.kernel]})")
    ms_pre = time_graph(prefill_plan, 20, 3)

    # ---- int16 prefill: the int16 contract (ActBlockQ16 rows) at config 4's shape,
    # quantize + lo / 256 hi operand layout + k_gemm_q4k_q16 on the f16 matrix cores
    def int16_prefill(i: int, st: int) -> None:
        dq.matmul_act(weights[i % ng], dq.ACT_Q16, xg, m, K, yf, N, None, st)

    log(f"int16 prefill M={m}")
    ms_q16 = time_graph(int16_prefill, 20, 3)
    ms_dec = time_graph(decode_plan(None), args.steps, args.warmup)
    ms_dec_x86 = time_graph(decode_plan(noqmm), args.steps, args.warmup)
    tpre = ops / (ms_pre * 1e-3) / 1e12
    dec_bytes = Q4K_ROW * N + 4 * K + 4 * N  # weights, the fp32 row, y

    log("ceilings: plain read at the GEMV's launch shape, int8 MFMA rate")
    ceil = ceilings(args.steps, args.warmup)
    read_ceiling = ceil["33MB"]["gbs"]
    mfma_ceiling = ceil["mfma"]["16x16x64"]["tops"]
    f16_ceiling = ceil["mfma"]["f16_32x32x16"]["tops"]

    traffic = measured_traffic()
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "ms_per_step_python_launches": round(ms_step_eager, 5),
        "timing": "HIP events around one replay of a HIP graph holding exactly `steps` steps (eager "
                  "warmup first); ms_per_step_python_launches is the same steps launched one by one "
                  "from Python",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: random valid Q4_K blocks (fp16 d/dmin in U(0.002,0.02)), x ~ N(0,1)",
        "config": {
            "workload": "config 3 gate/up decode step: dq_matmul M=1 (x -> Q8_K in-kernel, Q4_K GEMV), K=4096 N=14336",
            "weight_copies": nc,
            "weight_bytes": Q4K_ROW * N,
            "algorithmic_bytes_per_step": bytes_step,
        },
        "pct_peak_hbm": round(100 * value / PEAK_HBM_GBS, 2),
        "read_ceiling_gbs": read_ceiling,
        "pct_of_read_ceiling": round(100 * value / read_ceiling, 2),
        "best_read_gbs": ceil["read_shape_sweep"]["best_gbs"],
        "pct_of_best_read": round(100 * value / ceil["read_shape_sweep"]["best_gbs"], 2),
        "mfma_ceiling_tops": mfma_ceiling,
        "f16_mfma_ceiling_tflops": f16_ceiling,
        "ceilings": ceil,
        "tokens_per_s": round(1e3 / ms_step, 1),
        "roofline": {
            "kernel": "dq::k_gemv_slab<16, 2, true> (Q4_K x Q8_K, M=1, fused quantization, 56-row workgroups)",
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic.get("gemv_fused_m1"),
            "ms_per_launch": round(ms_step, 5),
        },
        "gemv_prequantized": {
            "kernel": "dq::k_gemv_slab<16, 2, false> (Q4_K x Q8_K, M=1; activations quantized by a separate launch)",
            "ms_per_launch": round(ms_gemv, 5),
            "gbs": round(bytes_step / (ms_gemv * 1e-3) / 1e9, 2),
        },
        "gemm": {
            "workload": f"config 4 prefill: Q4_K x Q8_K GEMM, M={m} K=4096 N=14336",
            "ms_per_launch": round(ms_gemm, 4),
            "tops": round(tops, 2),
            "matrix_core": "f16 (v_mfma_f32_32x32x16_f16 on exact integer operands)",
            "pct_peak_f16": round(100 * tops / PEAK_F16_TFLOPS, 2),
            "pct_of_f16_mfma_ceiling": round(100 * tops / f16_ceiling, 2),
            "tokens_per_s": round(m / (ms_gemm * 1e-3), 1),
            "roofline": {"kernel": "dq::k_gemm_q4k_h16 (ms per dq_gemm call: + k_act16_from_q8k)", "bound": "mfma",
                         "achieved": round(tops, 2), "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tops / PEAK_F16_TFLOPS, 4), "traffic": traffic.get("gemm_m512")},
        },
    }
    result["f32_expand_gemm"] = {
        "workload": f"config 4 prefill shape, fp32 activations: dq_matmul_plan (default plan -> kF32ExpandGemm), "
                    f"Q4_K M={m} K={K} N={N}",
        "ms_per_launch": round(ms_f32, 4),
        "tflops": round(tf32, 2),
        "ms_row_dot_gemv": round(ms_f32_rows, 4),
        "roofline": {"kernel": "dq::k_gemm_f32<Q4_K>", "bound": "mfma", "achieved": round(tf32, 2),
                     "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s", "frac": round(tf32 / PEAK_FP32_MFMA_TFLOPS, 4)},
    }
    result["prefill_default_plan"] = {
        "workload": f"config 4 prefill, M={m} K={K} N={N} Q4_K: dq_matmul_plan under KernelPlan's defaults with "
                    f"the engine's int8 row limit on a qmm-accelerated backend (unbounded) -> "
                    f"{dq.KERNEL_NAMES[sel_pre.kernel]} on per-32 activations",
        "ms_per_call": round(ms_pre, 4),
        "tflops": round(tpre, 2),
        "tokens_per_s": round(m / (ms_pre * 1e-3), 1),
        "roofline": {"kernel": "dq::k_gemm_q4k_p32 (ms per call: + per-32 quantize + k_act32_from_p32)",
                     "bound": "mfma", "achieved": round(tpre, 2), "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tpre / PEAK_F16_TFLOPS, 4), "traffic": traffic.get("prefill_default_m512")},
    }
    tq16 = ops / (ms_q16 * 1e-3) / 1e12
    result["prefill_int16_m512"] = {
        "workload": "config 4, M=512 K=4096 N=14336 Q4_K: dq_matmul_act(DQ_ACT_Q16) (int16 quantize, "
                    "k_act16i_from_q16, k_gemm_q4k_q16 on the f16 matrix cores)",
        "ms_per_call": round(ms_q16, 4), "tops": round(tq16, 1),
        "pct_peak_f16": round(100 * tq16 / PEAK_F16_TFLOPS, 2)}
    result["decode_default_plan"] = {
        "workload": f"config 3 decode, M=1 K={K} N={N} Q4_K: dq_matmul_plan under KernelPlan's defaults "
                    f"({dq.KERNEL_NAMES[sel_dec.kernel]}, per-32 activations quantized inside the GEMV: one launch)",
        "ms_per_call": round(ms_dec, 5),
        "gbs": round(dec_bytes / (ms_dec * 1e-3) / 1e9, 2),
        "roofline": {"kernel": "dq::k_gemv_slab<16, 0, true> (Q4_K x per-32, M=1, fused quantization, 56-row workgroups)", "bound": "hbm",
                     "achieved": round(dec_bytes / (ms_dec * 1e-3) / 1e9, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(dec_bytes / (ms_dec * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
        "without_qmm": {"kernel": dq.KERNEL_NAMES[sel_x86.kernel], "ms_per_call": round(ms_dec_x86, 5),
                        "gbs": round(dec_bytes / (ms_dec_x86 * 1e-3) / 1e9, 2),
                        "note": "the class cpu_baseline times (the reference's x86 default)"},
    }
    if ms_gated is not None:
        gbytes = 2 * Q4K_ROW * N + Q8K_ROW + 4 * N
        result["gated_m1"] = {
            "workload": "dq_matmul_gated(SiLU) M=1, Q4_K gate and up K=4096 N=14336 (one launch: "
                        "k_gemv<Q4_K, Q8_K, M=1, fused, gated>)",
            "ms_per_call": round(ms_gated, 5),
            "gbs": round(gbytes / (ms_gated * 1e-3) / 1e9, 2),
            "pct_peak_hbm": round(100 * gbytes / (ms_gated * 1e-3) / 1e9 / PEAK_HBM_GBS, 2),
            "ms_two_matmuls": round(ms_two, 5),
        }
    if args.sweep:
        result["prefill_sweep"] = prefill_sweep([int(v) for v in args.sweep.split(",")], weights, gen)
    if args.sweep:
        result["prefill_other_types_m512"] = prefill_other_types(gen)
    if args.stack_steps > 0:
        log(f"config 5 decode stack x{args.stack_steps}")
        result["decode_stack_m16"] = decode_stack(args.stack_steps, stream)
    if not args.no_cpu:
        log("CPU baseline")
        result["cpu_baseline"] = cpu_baseline(w_host, args.cpu_seconds)
        cpu_ms = result["cpu_baseline"].get("ms_per_call")
        if cpu_ms:
            result["decode_default_plan"]["without_qmm"]["speedup_vs_cpu_baseline"] = round(cpu_ms / ms_dec_x86, 2)
    result["output_checks"] = checks
    print(json.dumps(result), flush=True)
    if not all(v for key, v in checks.items() if key != "rows_checked"):
        raise SystemExit("output check failed: the timed kernels disagree with the GEMV on the same inputs")


if __name__ == "__main__":
    main()
