"""loom's drift spectrum, the classification its bridge suites print for every
accelerated layer (lucy/examples/apple/spectrum.go:8-70; used by
lucy/examples/apple/dispatch.go:34-167).

A difference `diff` (max |a - b| over a layer's outputs) against a tolerance
`tol` lands in one of seven buckets: FATAL (NaN/Inf), EXACT (0), INDUS
(<= tol), LOWBIT (<= 10 tol), DRIFT (<= 0.1), H-DRIFT (<= 1), BROKE.
"""
import math

import numpy as np

LABELS = ["EXACT", "INDUS", "LOWBIT", "DRIFT", "H-DRIFT", "BROKE", "FATAL"]
EXACT, INDUS, LOWBIT, DRIFT, H_DRIFT, BROKE, FATAL = range(7)


def classify(diff: float, tol: float) -> int:
    """classifyDrift (lucy/examples/apple/spectrum.go:37-58)."""
    if math.isnan(diff) or math.isinf(diff):
        return FATAL
    if diff == 0:
        return EXACT
    if diff <= tol:
        return INDUS
    if diff <= tol * 10:
        return LOWBIT
    if diff <= 0.1:
        return DRIFT
    if diff <= 1.0:
        return H_DRIFT
    return BROKE


def infer_tolerance(dtype: str) -> float:
    """inferDriftTolerance (lucy/examples/apple/spectrum.go:60-70)."""
    return {"FP32": 1e-7, "FP16": 1e-5, "INT16": 1e-3, "INT8": 1e-3, "INT4": 1e-3}.get(dtype, 1e-7)


def parity_tolerance(dtype: str) -> float:
    """parityTolerance (lucy/examples/apple/dispatch.go:240-255)."""
    return {"FP32": 1e-2, "FP16": 5e-2, "INT16": 0.5, "INT8": 2.0, "INT4": 4.0}.get(dtype, 1e-2)


def gpu_parity_tolerance(dtype: str) -> float:
    """The accelerator-GPU parity bar of runDispatchCase: max(10 tol, 0.05)
    (lucy/examples/apple/dispatch.go:155-159)."""
    return max(parity_tolerance(dtype) * 10, 0.05)


def max_abs_diff(a: np.ndarray, b: np.ndarray) -> float:
    """maxAbsDiffTensor for float32 tensors (lucy/examples/apple/dispatch.go:205-238):
    the difference is taken in fp32, its magnitude in fp64; a length
    mismatch is MaxFloat64.  The running maximum starts at 0 and takes a
    difference only when `d > m`, so NaN differences never enter it."""
    a = np.asarray(a, np.float32).ravel()
    b = np.asarray(b, np.float32).ravel()
    if a.size != b.size:
        return float(np.finfo(np.float64).max)
    with np.errstate(invalid="ignore", over="ignore"):
        d = np.abs((a - b).astype(np.float64))
    d = d[~np.isnan(d)]
    return float(d.max()) if d.size else 0.0


def histogram(a: np.ndarray, b: np.ndarray, tol: float) -> list[int]:
    """Every output element classified on its own |a - b| (fp32 difference,
    as maxAbsDiffTensor forms it): counts per bucket, in LABELS order."""
    a = np.asarray(a, np.float32).ravel()
    b = np.asarray(b, np.float32).ravel()
    with np.errstate(invalid="ignore", over="ignore"):
        d = np.abs((a - b).astype(np.float64))
    counts = [0] * 7
    counts[FATAL] = int(np.count_nonzero(~np.isfinite(d)))
    f = d[np.isfinite(d)]
    counts[EXACT] = int(np.count_nonzero(f == 0))
    counts[INDUS] = int(np.count_nonzero((f > 0) & (f <= tol)))
    counts[LOWBIT] = int(np.count_nonzero((f > tol) & (f <= 10 * tol)))
    counts[DRIFT] = int(np.count_nonzero((f > 10 * tol) & (f <= 0.1)))
    counts[H_DRIFT] = int(np.count_nonzero((f > 0.1) & (f <= 1.0)))
    counts[BROKE] = int(np.count_nonzero(f > 1.0))
    return counts
