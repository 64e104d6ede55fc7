"""The reference-side binding (dynalm_amd/integration/dynaq_cpu_shim.cpp) compiles
against dynacore's own headers: ExternalMatmulKernel, CpuDevice::kernel_plan and
register_external_matmul (dynacore/include/dynacore/cpu/cpu_device.h:22-72), KernelPlan
(kernel_plan.h) and Status (base/status.h), with include/dynaq.h. Runs where the
reference tree is present (this container); compiling needs no GPU."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INC = "/root/reference/dynacore/include"
SHIM = os.path.join(ROOT, "dynalm_amd", "integration", "dynaq_cpu_shim.cpp")


@pytest.mark.skipif(not os.path.isdir(REF_INC) or shutil.which("g++") is None,
                    reason="needs the reference's headers and g++")
def test_shim_compiles_against_reference_headers(tmp_path):
    obj = tmp_path / "shim.o"
    cmd = ["g++", "-std=c++20", "-O1", "-Wall", "-Werror", "-c", SHIM, "-o", str(obj),
           "-DENGINE_HAS_AVX2=1", "-DENGINE_HAS_AVX512=0", "-DENGINE_HAS_AMX=0", "-DENGINE_HAS_NEON=0",
           f"-I{REF_INC}", f"-I{os.path.join(ROOT, 'include')}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    syms = subprocess.run(["nm", "-C", str(obj)], capture_output=True, text=True).stdout
    # the shim calls exactly these entry points of the library
    for name in ("dq_external_create", "dq_external_set_plan", "dq_external_run", "dq_external_eligible"):
        assert f"U {name}" in syms, name
    assert "dynaq_shim::register_dynaq" in syms
