"""Contract error metrics (reference src/xpu/error_metric.py:19-29).

``max_rel_error`` is the reference's peak-normalised component-wise error:
max(max(|dRe|, |dIm|)) / max|ref|, ``inf`` for any non-finite value.
``rel_l2`` is the relative L2 error the MI355X build gates on (<= 1e-5).
"""
from __future__ import annotations

import numpy as np


def max_rel_error(got, ref) -> float:
    g = np.asarray(got)
    r = np.asarray(ref)
    delta = np.maximum(np.abs(g.real - r.real), np.abs(g.imag - r.imag))
    scale = np.abs(r).max() if r.size else 0.0
    if not np.isfinite(delta).all() or not np.isfinite(scale):
        return float("inf")
    if delta.size == 0:
        return 0.0
    return float(delta.max() / max(float(scale), 1e-12))


def rel_l2(got, ref) -> float:
    g = np.asarray(got, dtype=np.complex128)
    r = np.asarray(ref, dtype=np.complex128)
    d = float(np.linalg.norm((g - r).ravel()))
    s = float(np.linalg.norm(r.ravel()))
    if not np.isfinite(d) or not np.isfinite(s):
        return float("inf")
    return d / max(s, 1e-300)
