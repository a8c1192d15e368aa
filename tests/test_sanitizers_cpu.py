"""The GGUF reader (untrusted input: ziglm_amd/csrc/gguf.cpp) and the CPU oracle built with
AddressSanitizer and UndefinedBehaviorSanitizer (host compilers, tests/asan/Makefile), and the
suites that exercise them run against those builds in a child process: the GGUF reference
tests, every reject path, the differential test against oracle/gguf_ref.py (random files,
every truncation point, 1,500 byte-mutated files), and the oracle's pinning suites. Any
sanitizer report fails the run (halt_on_error, no recovery from undefined behaviour)."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _runtime(name):
    p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


@pytest.fixture(scope="module")
def asan_build(tmp_path_factory):
    if not shutil.which("g++") or not shutil.which("gcc") or not _runtime("libasan.so"):
        pytest.skip("host compilers with AddressSanitizer are not available")
    if not os.path.exists("/opt/rocm/lib/libamdhip64.so"):
        pytest.skip("HIP runtime not installed")
    out = tmp_path_factory.mktemp("asan")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "asan"), f"OUT={out}"], check=True,
                   capture_output=True, text=True)
    return out


def test_gguf_reader_and_oracle_under_asan_ubsan(asan_build):
    env = dict(os.environ)
    env.update({
        "HIP_BRIDGE_LIB": str(asan_build / "libzl_gguf_asan.so"),
        "ZIGLM_ORACLE_LIB": str(asan_build / "liboracle_asan.so"),
        "LD_PRELOAD": " ".join(p for p in (_runtime("libasan.so"), _runtime("libubsan.so")) if p),
        # the interpreter itself is not instrumented: its own allocations are not leaks to report
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
    })
    tests = ["tests/test_gguf_cpu.py", "tests/test_oracle_cpu.py", "tests/test_oracle_gemv_cpu.py",
             "tests/test_model_ref_cpu.py"]
    p = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu",
                        *tests], cwd=ROOT, env=env, capture_output=True, text=True, timeout=1500)
    log = p.stdout + p.stderr
    assert "ERROR: AddressSanitizer" not in log and "runtime error:" not in log, log[-6000:]
    assert p.returncode == 0, log[-6000:]
    assert " passed" in log
