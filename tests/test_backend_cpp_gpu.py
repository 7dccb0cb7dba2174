"""Runs the C++ tests of RocmBackend (tests/cpp/test_rocm_backend.cpp): the
IBackend::attention-shaped layer (backend.h:105-110) over the C-ABI, checked
against the CPU oracle -- mask forms, strides, scale, causal, the
reference's exception types, and hipGraph capture with a reserved
workspace.  The binary is built by __graft_entry__.build()."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_rocm_backend")


def test_rocm_backend_cpp():
    assert os.path.exists(BIN), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL PASSED" in r.stdout
