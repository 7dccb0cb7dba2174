"""Tolerance helpers shared by the tests.

bf16 kernels are compared with the fp32 oracle on the kernel's fp32 output:
max-abs <= 2e-2 and mean-rel <= 1e-3, where mean-rel = sum|got-ref| / sum|ref|
(robust to reference values near zero).
"""
import numpy as np

MAX_ABS = 2e-2
MEAN_REL = 1e-3


def mean_rel(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(got - ref).sum() / max(np.abs(ref).sum(), 1e-300))


def assert_close_bf16(got, ref, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    mx = float(np.abs(got - ref).max()) if got.size else 0.0
    mr = mean_rel(got, ref) if got.size else 0.0
    assert mx <= MAX_ABS and mr <= MEAN_REL, f"{what}: max-abs {mx:.3e}, mean-rel {mr:.3e}"
    return mx, mr


def cosine(got, ref):
    """Cosine similarity of the flattened arrays (the reference's alignment
    metric, tests/alignment/test_rdt1b_alignment.py:287-299, 426)."""
    g = np.asarray(got, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    return float(g @ r / max(np.linalg.norm(g) * np.linalg.norm(r), 1e-300))
