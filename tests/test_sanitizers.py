"""Host sanitizer run (CPU only): builds tests/cpp/sanitize_host.cpp with
gcc/g++ -fsanitize=address,undefined and runs it.  It drives the safetensors
header parser and sf_safetensors_inspect (servoflow_amd/host/st_format.cpp;
the reference's SafeTensorsLoader::parse_header / inspect,
src/loader/safetensors.cpp:62-114) through valid, truncated, mutated and
hostile headers, the loader's element conversions, and every function of
the CPU oracle (oracle/sf_oracle.c) on small ragged shapes.  An
out-of-bounds access, leak or undefined behaviour aborts the binary, which
fails the test with the sanitizer report."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")


@pytest.mark.skipif(shutil.which("g++") is None or shutil.which("gcc") is None, reason="gcc/g++ not found")
def test_host_code_under_asan_ubsan():
    b = subprocess.run(["make", "-s", "-C", CPP, "sanitize"], capture_output=True, text=True, timeout=300)
    assert b.returncode == 0, b.stdout + b.stderr
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=23",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([os.path.join(CPP, "_build", "sanitize_host")], capture_output=True, text=True,
                       timeout=300, env=env)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert "all checks passed" in r.stdout
