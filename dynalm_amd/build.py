"""Builds libdynaq.so (the C-ABI library) in-tree with hipcc for gfx950, and
libdqceil.so, the benchmark's ceiling probes (a plain read at the decode GEMV's
launch shape and an int8 MFMA rate loop; bench.py loads it, the library does not).

    python -m dynalm_amd.build          # or dynalm_amd.build.build()

The library has no torch types in its interface; PyTorch is not needed to build it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libdynaq.so")
CEIL_LIB = os.path.join(LIB_DIR, "libdqceil.so")
CEIL_SOURCES = ["dq_ceiling.hip"]

SOURCES = ["dq_kernels.hip", "dq_gemv.hip", "dq_gemm.hip", "dq_gemm_b32.hip", "dq_gemm_f32.hip", "dq_gemm_h16.hip", "dq_gemm_p32.hip", "dq_gemm_q16.hip", "dq_gemm_q6x.hip", "dq_skinny.hip", "dq_api.cpp",
           "dq_gguf.cpp", "dq_external.cpp", "dq_noalloc.hip",
           "dq_plan.cpp"]
ARCH = os.environ.get("DYNAQ_ARCH", "gfx950")

# Device code: IEEE fp32 division/sqrt (the quantizers need correctly rounded
# amax / 127 and 1 / d), no FMA contraction (float steps round where written),
# no packed-fp32 instructions.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(cc: str, src: str, verbose: bool) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(LIB_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [cc, *HIP_FLAGS, "-x", "hip", "-c", path, "-o", obj, f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{out}")
    if out.strip() and verbose:
        print(out)
    return obj


def build(verbose: bool = False) -> str:
    from concurrent.futures import ThreadPoolExecutor

    os.makedirs(LIB_DIR, exist_ok=True)
    cc = hipcc()
    srcs = SOURCES + CEIL_SOURCES
    with ThreadPoolExecutor(max_workers=len(srcs)) as pool:
        objs = dict(zip(srcs, pool.map(lambda src: _compile(cc, src, verbose), srcs)))
    for lib, group in ((LIB, SOURCES), (CEIL_LIB, CEIL_SOURCES)):
        tmp = lib + ".tmp"
        cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *(objs[s] for s in group)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
        os.replace(tmp, lib)
    for o in objs.values():
        os.remove(o)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
