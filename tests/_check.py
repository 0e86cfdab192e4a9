"""Tolerance checks shared by the parity tests.

fp32: |y - y_ref| <= 1e-5 * sum_j |a_ij * x_j| per output element (the
hot path's stated bound), with y_ref the sequential fp32 oracle.
bf16 MFMA paths: relative L2 error <= 1e-2 against the fp32 oracle.
"""
import numpy as np

FP32_REL = 1e-5
BF16_REL_L2 = 1e-2


def assert_within_bound(y, ref, bound, rel=FP32_REL, what="output"):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    bound = np.asarray(bound, np.float64)
    assert y.shape == ref.shape, (y.shape, ref.shape)
    assert np.all(np.isfinite(y)), f"{what}: non-finite values"
    err = np.abs(y - ref)
    tol = rel * bound
    bad = err > tol
    if bad.any():
        i = np.flatnonzero(bad.ravel())[:5]
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} elements exceed "
            f"{rel:g}*sum|a*x|; first {i.tolist()}: got "
            f"{y.ravel()[i].tolist()} want {ref.ravel()[i].tolist()} "
            f"tol {tol.ravel()[i].tolist()}")


def rel_l2(y, ref):
    y = np.asarray(y, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    return float(np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-300))
