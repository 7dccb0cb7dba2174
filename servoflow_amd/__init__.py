"""servoflow_amd — MI355X-native attention hot path of servoflow's RDT-1B denoise loop.

Kernels live in lib/libsf_hip_kernels.so (C-ABI: include/sf_hip.h), built
from csrc/ for gfx950.  `abi` holds the ctypes bindings; `attention` is the
torch-tensor front end used by the tests and the benchmark.
"""
from . import abi  # noqa: F401

__all__ = ["abi"]
