"""Contract error metrics (reference src/xpu/error_metric.py:19-29).

``max_rel_error`` is the reference's correctness contract: the peak-
normalised component-wise deviation

    max(max(|Re(got - ref)|, |Im(got - ref)|)) / max|ref|

computed with element-wise NumPy operations, so a NaN in either component
(which Python's builtin ``max`` would swallow) scores ``inf``; any non-finite
deviation or reference scores ``inf``.  The reference's gate is < 1e-4.

``rel_l2`` is the relative L2 error ||got - ref|| / ||ref|| in float64, the
metric this library gates its own kernels on (<= 1e-5), also ``inf`` for
non-finite input.
"""
from __future__ import annotations

import numpy as np


def max_rel_error(got, ref) -> float:
    """Contract error between ``got`` and ``ref``; ``inf`` if non-finite."""
    g = np.asarray(got)
    r = np.asarray(ref)
    delta = np.maximum(np.abs(g.real - r.real), np.abs(g.imag - r.imag))
    if delta.size == 0:
        return 0.0
    scale = np.abs(r).max()
    if not np.isfinite(delta).all() or not np.isfinite(scale):
        return float("inf")
    return float(delta.max() / max(float(scale), 1e-12))


def rel_l2(got, ref) -> float:
    """||got - ref||_2 / ||ref||_2 in float64; ``inf`` if non-finite."""
    g = np.asarray(got, dtype=np.complex128).ravel()
    r = np.asarray(ref, dtype=np.complex128).ravel()
    d = float(np.linalg.norm(g - r))
    s = float(np.linalg.norm(r))
    if not np.isfinite(d) or not np.isfinite(s):
        return float("inf")
    if d == 0.0:
        return 0.0
    return d / max(s, 1e-300)
