"""CPU oracle for the complex64 FFT hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker or the
timed CPU baseline.  The shipped library never routes through it.

It restates the reference's algorithm for this path in float64:

* the radix-2 DIT/DIF core of ``include/butterfly/fft.hpp:28-96`` (C, in
  ``butterfly_oracle.c``, loaded through ctypes from ``oracle/_build``);
* the wrapper semantics of ``src/xpu/entry.py`` around that core:
  norm table ``norm_scale`` (entry.py:81-102), inverse by conjugation
  (entry.py:617-628), the dedicated real flows (entry.py:555-587 with the
  formulas of kernels.py:1127-1258 / runner.py:1776-1834) and the
  Hermitian rebuild of the compatibility C2R path (entry.py:671-696);
* the contract error metric ``max_rel_error`` (src/xpu/error_metric.py:19-29).

How each function is pinned (tests/test_oracle.py):

=========================  =================================================
function                   pinned against
=========================  =================================================
bit_reverse                reference KAT {0,4,2,6,1,5,3,7} (fft_check.cpp:43-54),
                           the reference's own ref_bit_reverse (oracle/_ref)
fft_dit / fft_dif          naive O(N^2) DFT, numpy.fft, the reference's own
                           butterfly::fft_dit/fft_dif built into oracle/_ref
                           (bit-exact), KAT input of fft_check.cpp:56-76,
                           impulse/tone (test_fft.py:196-211), DC sentinel
c2c (inverse, norms)       numpy.fft.fft/ifft with every norm, round trip
r2c_dedicated / c2r_*      numpy.fft.rfft/irfft, DC/Nyquist-imaginary
                           independence, Hermitian symmetry
four_step                  numpy.fft (closed form of the Bailey split)
max_rel_error              closed-form hand-computed cases
=========================  =================================================
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libref_butterfly.so")

_lib = None
_ref = None

NORMS = ("none", "forward", "backward", "ortho")


def build() -> None:
    """Compile the C restatement (and the reference shim when its tree exists)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        dp = ctypes.POINTER(ctypes.c_double)
        lib.oracle_bit_reverse.argtypes = [ctypes.c_uint32, ctypes.c_int]
        lib.oracle_bit_reverse.restype = ctypes.c_uint32
        lib.oracle_fft_dit.argtypes = [dp, ctypes.c_int64]
        lib.oracle_fft_dif.argtypes = [dp, ctypes.c_int64]
        lib.oracle_fft_batch.argtypes = [dp, ctypes.c_int64, ctypes.c_int64,
                                         ctypes.c_int, ctypes.c_int]
        lib.oracle_time_fft_batch.argtypes = [dp, ctypes.c_int64, ctypes.c_int64,
                                              ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.oracle_time_fft_batch.restype = ctypes.c_double
        lib.oracle_naive_dft.argtypes = [dp, dp, ctypes.c_int64, ctypes.c_int]
        _lib = lib
    return _lib


def reference_lib():
    """The reference's own CPU FFT compiled into oracle/_ref, or None."""
    global _ref
    if _ref is None and os.path.exists(_REF_PATH):
        lib = ctypes.CDLL(_REF_PATH)
        dp = ctypes.POINTER(ctypes.c_double)
        lib.ref_fft_batch.argtypes = [dp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int]
        lib.ref_time_fft_batch.argtypes = [dp, ctypes.c_int64, ctypes.c_int64,
                                           ctypes.c_int, ctypes.c_int]
        lib.ref_time_fft_batch.restype = ctypes.c_double
        if hasattr(lib, "ref_time_fft_batch_mt"):
            lib.ref_time_fft_batch_mt.argtypes = [dp, ctypes.c_int64, ctypes.c_int64,
                                                  ctypes.c_int, ctypes.c_int, ctypes.c_int]
            lib.ref_time_fft_batch_mt.restype = ctypes.c_double
        lib.ref_bit_reverse.argtypes = [ctypes.c_uint, ctypes.c_int]
        lib.ref_bit_reverse.restype = ctypes.c_uint
        _ref = lib
    return _ref


def _dptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def _rows(x) -> tuple[np.ndarray, bool]:
    a = np.array(x, dtype=np.complex128, copy=True, order="C")
    squeeze = a.ndim == 1
    return (a[None, :] if squeeze else a), squeeze


def bit_reverse(i: int, bits: int) -> int:
    """bit_reverse.hpp:15-22."""
    return int(_load().oracle_bit_reverse(i, bits))


def _core(x, dif: bool):
    a, squeeze = _rows(x)
    n = a.shape[-1]
    if n & (n - 1) or n <= 0:
        raise ValueError(f"oracle core needs a power-of-two length, got {n}")
    rc = _load().oracle_fft_batch(_dptr(a), n, a.shape[0], int(dif), 1)
    if rc != 0:
        raise ValueError("oracle_fft_batch failed")
    return a[0] if squeeze else a


def fft_dit(x):
    """Forward FFT over the last axis, fft.hpp:70-80 (radix-2 DIT, float64)."""
    return _core(x, False)


def fft_dif(x):
    """Forward FFT over the last axis, fft.hpp:84-96 (radix-2 DIF, float64)."""
    return _core(x, True)


def reference_fft(x, dif: bool = False):
    """The reference's own butterfly::fft_dit/fft_dif (oracle/_ref), or None."""
    lib = reference_lib()
    if lib is None:
        return None
    a, squeeze = _rows(x)
    rc = lib.ref_fft_batch(_dptr(a), a.shape[-1], a.shape[0], int(dif))
    if rc != 0:
        raise ValueError("ref_fft_batch failed")
    return a[0] if squeeze else a


def naive_dft(x, inverse: bool = False):
    """O(N^2) DFT, fft_check.cpp:20-34 restated (brute-force truth)."""
    a, squeeze = _rows(x)
    out = np.empty_like(a)
    for r in range(a.shape[0]):
        row = np.ascontiguousarray(a[r])
        o = np.empty_like(row)
        _load().oracle_naive_dft(_dptr(row), _dptr(o), row.shape[0], int(inverse))
        out[r] = o
    return out[0] if squeeze else out


def norm_scale(n: int, transform_direction: str, norm: str) -> float:
    """entry.py:81-102 (torch.fft norm table)."""
    if transform_direction not in ("forward", "inverse"):
        raise ValueError(f"bad transform_direction {transform_direction!r}")
    if norm not in NORMS:
        raise ValueError(f"bad norm {norm!r}")
    if norm == "ortho":
        return 1.0 / math.sqrt(n)
    if (norm == "forward" and transform_direction == "forward") or (
            norm == "backward" and transform_direction == "inverse"):
        return 1.0 / n
    return 1.0


def c2c(x, transform_direction: str = "forward", norm: str = "backward",
        decomposition: str = "dit"):
    """C2C with the reference's wrapper semantics (entry.py:617-628): the
    inverse conjugates the input, runs the forward core and conjugates the
    output; the norm's epilogue scale is applied last."""
    a, squeeze = _rows(x)
    n = a.shape[-1]
    core = fft_dif if decomposition == "dif" else fft_dit
    inv = transform_direction == "inverse"
    y = core(np.conj(a) if inv else a)
    if inv:
        y = np.conj(y)
    y = y * norm_scale(n, transform_direction, norm)
    return y[0] if squeeze else y


def r2c_dedicated(x, norm: str = "backward", decomposition: str = "dit"):
    """R2C dedicated half-length flow (entry.py:567-577): pack
    z[k] = x[2k] + i*x[2k+1], run the N/2-point forward core, then the
    stitch of kernels.py:1127-1177 with the norm scale fused:
    a = (Z[k] + conj Z[j])/2, c = (Z[k] - conj Z[j])/2, j = (N/2-k) % (N/2),
    X[k] = a - i*w*c, w = exp(-2*pi*i*k/N); DC/Nyquist imaginary = 0."""
    a = np.asarray(x, dtype=np.float64)
    squeeze = a.ndim == 1
    a2 = a[None, :] if squeeze else a
    n = a2.shape[-1]
    n2 = n // 2
    z = a2[:, 0::2] + 1j * a2[:, 1::2]
    core = fft_dif if decomposition == "dif" else fft_dit
    Z = core(z) if n2 > 0 else z
    k = np.arange(n2 + 1)
    zk = Z[:, k % n2]
    zj = Z[:, (n2 - k) % n2]
    av = 0.5 * (zk + np.conj(zj))
    cv = 0.5 * (zk - np.conj(zj))
    w = np.exp(-2j * np.pi * k / n)
    X = av - 1j * w * cv
    X[:, 0] = X[:, 0].real
    X[:, n2] = X[:, n2].real
    X = np.ascontiguousarray(X * norm_scale(n, "forward", norm))
    return X[0] if squeeze else X


def c2r_dedicated(xh, n: int, norm: str = "backward", decomposition: str = "dit"):
    """C2R dedicated half-length flow (entry.py:578-587): pre-twiddle of
    kernels.py:1180-1229 (DC/Nyquist imaginary parts ignored), the direct
    N/2-point core, then the mirror/scale unpack of kernels.py:1232-1258 with
    scale = 2*norm_scale(N, inverse, norm)."""
    h = np.asarray(xh, dtype=np.complex128)
    squeeze = h.ndim == 1
    h2 = (h[None, :] if squeeze else h).copy()
    n2 = n // 2
    if h2.shape[-1] != n2 + 1:
        raise ValueError(f"half spectrum must have N/2+1={n2 + 1} bins")
    h2[:, 0] = h2[:, 0].real
    h2[:, n2] = h2[:, n2].real
    k = np.arange(n2)
    xk = h2[:, k]
    xj = h2[:, n2 - k]
    av = 0.5 * (xk + np.conj(xj))
    cv = 0.5 * (xk - np.conj(xj))
    w = np.exp(2j * np.pi * k / n)
    Z = av + 1j * w * cv
    core = fft_dif if decomposition == "dif" else fft_dit
    u = core(Z)
    m = (n2 - k) % n2
    um = u[:, m] * (2.0 * norm_scale(n, "inverse", norm))
    out = np.empty((h2.shape[0], n), dtype=np.float64)
    out[:, 0::2] = um.real
    out[:, 1::2] = um.imag
    out = np.ascontiguousarray(out)
    return out[0] if squeeze else out


def hermitian_reconstruct(xh, n: int):
    """entry.py:671-696: full spectrum from a half spectrum, mirroring
    X[n-k] = conj X[k] with DC/Nyquist imaginary parts zeroed."""
    h = np.asarray(xh, dtype=np.complex128)
    squeeze = h.ndim == 1
    h2 = h[None, :] if squeeze else h
    m = n // 2 + 1
    full = np.empty((h2.shape[0], n), dtype=np.complex128)
    full[:, :m] = h2
    tail = h2[:, 1:m - 1] if n % 2 == 0 else h2[:, 1:m]
    full[:, m:] = np.conj(tail[:, ::-1])
    full[:, 0] = full[:, 0].real
    if n % 2 == 0:
        full[:, m - 1] = full[:, m - 1].real
    return full[0] if squeeze else full


def c2r_compat(xh, n: int, norm: str = "backward"):
    """Compatibility C2R of entry.py:603-616: Hermitian rebuild, inverse C2C
    through the conjugate trick, real part."""
    full = hermitian_reconstruct(xh, n)
    return c2c(full, "inverse", norm).real


def four_step(x, n1: int, n2: int, transform_direction: str = "forward"):
    """Bailey 4-step split N = n1*n2 (adapter_hybrid.py:224-270 semantics):
    column FFTs of length n1, twiddle W_N^(n2*k1), row FFTs of length n2,
    output X[k1 + n1*k2]; sub-FFTs by the oracle core."""
    a, squeeze = _rows(x)
    n = n1 * n2
    if a.shape[-1] != n:
        raise ValueError("n1*n2 must equal the row length")
    inv = transform_direction == "inverse"
    src = np.conj(a) if inv else a
    cols = src.reshape(-1, n1, n2).transpose(0, 2, 1)          # [b, n2, n1]
    y = fft_dit(cols.reshape(-1, n1)).reshape(-1, n2, n1)
    k1 = np.arange(n1)
    tw = np.exp(-2j * np.pi * np.outer(np.arange(n2), k1) / n)
    y = y * tw[None]
    rows = y.transpose(0, 2, 1).reshape(-1, n2)                # [b, k1, n2]
    z = fft_dit(rows).reshape(-1, n1, n2)                       # [b, k1, k2]
    out = z.transpose(0, 2, 1).reshape(-1, n)                   # X[k1 + n1*k2]
    if inv:
        out = np.conj(out)
    return out[0] if squeeze else out


def max_rel_error(got, ref) -> float:
    """error_metric.py:19-29: max(max(|dRe|, |dIm|)) / max|ref|; inf if not finite."""
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
    """||got - ref||_2 / ||ref||_2 (inf when not finite)."""
    g = np.asarray(got, dtype=np.complex128)
    r = np.asarray(ref, dtype=np.complex128)
    d = np.linalg.norm((g - r).ravel())
    s = np.linalg.norm(r.ravel())
    if not np.isfinite(d) or not np.isfinite(s):
        return float("inf")
    return float(d / max(s, 1e-300))


def time_cpu_fft(x, threads: int = 1, reps: int = 5, use_reference: bool = True):
    """Median seconds of the reference CPU path (oracle/_ref when built,
    else the C restatement) over the rows of ``x``; returns (seconds, kind)."""
    a, _ = _rows(x)
    n, b = a.shape[-1], a.shape[0]
    lib = reference_lib() if use_reference else None
    if lib is not None and threads <= 1:
        return float(lib.ref_time_fft_batch(_dptr(a), n, b, 0, reps)), "reference"
    if lib is not None and hasattr(lib, "ref_time_fft_batch_mt"):
        return float(lib.ref_time_fft_batch_mt(_dptr(a), n, b, 0, reps, threads)), "reference"
    return float(_load().oracle_time_fft_batch(_dptr(a), n, b, 0, threads, reps)), "port"
