"""The host C++ under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

tests/sanitize/Makefile builds libdynaq_san.so: dq_gguf.cpp, dq_api.cpp,
dq_external.cpp and dq_plan.cpp compiled by g++ with -fsanitize=address,undefined
(errors abort), linked with the HIP sources. A child Python process with the ASan
runtime preloaded and DYNAQ_LIB pointing at it runs the CPU tests of the GGUF reader
(every truncation, seeded mutations, malformed headers), kernel selection, the C-ABI
argument validation and the external adapter's shape rules; they must pass with no
sanitizer report. A planted heap overread in a separate probe library shows the
harness reports what it should."""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_DIR = os.path.join(ROOT, "tests", "sanitize")
SAN_LIB = os.path.join(SAN_DIR, "_build", "libdynaq_san.so")
PLANTED = os.path.join(SAN_DIR, "_build", "libplanted.so")
TESTS = ["tests/test_gguf.py", "tests/test_plan.py", "tests/test_abi.py", "tests/test_external.py"]


def _runtime(name: str) -> str | None:
    if shutil.which("g++") is None:
        return None
    p = subprocess.run(["g++", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


@pytest.fixture(scope="module")
def san_env():
    asan = _runtime("libasan.so")
    if asan is None or not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("needs g++ with libasan and hipcc")
    r = subprocess.run(["make", "-C", SAN_DIR, "-s", "-j8"], capture_output=True, text=True, timeout=1200)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    env = dict(os.environ)
    env.update(LD_PRELOAD=asan, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", DYNAQ_LIB=SAN_LIB, PYTHONDONTWRITEBYTECODE="1")
    return env


def test_host_code_clean_under_sanitizers(san_env):
    probe = ("import dynalm_amd as dq; dq.lib(); m = open('/proc/self/maps').read(); "
             "print('libdynaq_san.so' in m, 'libasan' in m, '/lib/libdynaq.so' in m)")
    r = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env=san_env, capture_output=True, text=True,
                       timeout=120)
    assert r.stdout.split() == ["True", "True", "False"], r.stdout + r.stderr[-2000:]
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu", *TESTS],
                       cwd=ROOT, env=san_env, capture_output=True, text=True, timeout=1200)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert " passed" in r.stdout


def test_harness_reports_a_planted_overread(san_env):
    code = f"import ctypes; ctypes.CDLL({PLANTED!r}).dqsan_planted_oob(4)"
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=san_env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert "heap-buffer-overflow" in r.stderr, r.stderr[-2000:]
