"""Host-side matrices of the reference's M2 and M3 flows (reference
src/xpu/matrices.py:64-405), numpy only (no torch).

* ``local_matrix(tile, direction)``: the linear map of the block-local
  radix-2 stages of one ``tile``-point block.  Its coefficients depend only
  on ``tile``, and in closed form it is
    DIT: ``M = F_T @ P``  (applied to the bit-reversed block: ``M @ bitrev(x) = fft(x)``)
    DIF: ``M = P @ F_T``  (followed by the bit-reversed output: ``bitrev(M @ x) = fft(x)``)
  with ``F_T`` the ``tile``-point DFT matrix and ``P`` the bit-reversal
  permutation (its own inverse).  This module builds it that way.
* ``tail_group_table(n0, glog, direction)``: ``glog`` consecutive global
  stages (half-spans ``n0, 2 n0, ...``) as one map on each period-``P``
  block, ``P = n0 << glog``, read out at XOR offsets:
  ``out[i] = sum_k table[k, i mod P] * in[i ^ (k * n0)]``.
* ``tail_groups``: the greedy partition of the tail stages into such groups
  and single stages.

On MI355X these are not what the kernels run: the dense-dot flow builds
its DFT-8 factors on the device, and the M3 names run the LDS / four-step
kernels.  The functions keep the reference's names, signatures and layouts
(planar float32 ``[k, i]`` / transposed ``MT``) for callers and scripts that
use them, and ``verify_*`` check them against independent stage loops.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "local_matrix",
    "local_matrix_planar",
    "verify_local_matrix",
    "verify_decomposition",
    "tail_group_table",
    "tail_group_planar",
    "apply_tail_group_table",
    "verify_tail_group",
    "verify_grouped_decomposition",
    "tail_groups",
]


def _log2_exact(n: int) -> int:
    if not isinstance(n, (int, np.integer)) or n <= 0 or (n & (n - 1)) != 0:
        raise ValueError(f"expected a power of two, got {n}")
    return int(n).bit_length() - 1


def _bitrev(n: int) -> np.ndarray:
    """i -> bit reversal of i over log2(n) bits, as an index array."""
    bits = _log2_exact(n)
    i = np.arange(n)
    r = np.zeros(n, dtype=np.int64)
    for b in range(bits):
        r |= ((i >> b) & 1) << (bits - 1 - b)
    return r


def _dft(n: int) -> np.ndarray:
    k = np.arange(n)
    return np.exp(-2j * np.pi * np.outer(k, k) / n)


def _direction(direction: str) -> str:
    if direction not in ("dit", "dif"):
        raise ValueError(f"unknown direction {direction!r}")
    return direction


def local_matrix(tile: int, direction: str = "dit") -> np.ndarray:
    """complex128 ``M`` (``tile`` x ``tile``) with ``out = M @ in`` for the
    local group: DIT ``F_T P`` (input in bit-reversed order), DIF ``P F_T``
    (output in bit-reversed order)."""
    _log2_exact(tile)
    _direction(direction)
    f = _dft(tile)
    br = _bitrev(tile)
    return f[:, br] if direction == "dit" else f[br, :]


def local_matrix_planar(tile: int, direction: str = "dit"):
    """``(MT_r, MT_i)`` float32, C-contiguous, of ``MT = M.T`` (the
    row-vector convention ``out_row = in_row @ MT``)."""
    mt = local_matrix(tile, direction).T
    return np.ascontiguousarray(mt.real, dtype=np.float32), np.ascontiguousarray(mt.imag, dtype=np.float32)


def _stage(v: np.ndarray, half: int, direction: str) -> np.ndarray:
    """One radix-2 stage of half-span ``half`` over blocks of ``2 half``,
    pair by pair; its twiddle is exp(-2 pi i j / (2 half)) for j < half."""
    out = np.empty_like(v)
    size = v.shape[0]
    for base in range(0, size, 2 * half):
        for j in range(half):
            w = np.exp(-1j * np.pi * j / half)
            a, b = v[base + j], v[base + j + half]
            if direction == "dit":
                out[base + j], out[base + j + half] = a + w * b, a - w * b
            else:
                out[base + j], out[base + j + half] = a + b, (a - b) * w
    return out


def _local_stages(v: np.ndarray, tile: int, direction: str) -> np.ndarray:
    logt = _log2_exact(tile)
    halves = [1 << s for s in range(logt)]
    for h in halves if direction == "dit" else halves[::-1]:
        v = _stage(v, h, direction)
    return v


def verify_local_matrix(tile: int, direction: str = "dit", rtol=1e-10, atol=1e-12) -> float:
    """Max abs difference between ``local_matrix`` (closed form) and the
    block-local stages applied one pair at a time to each unit vector;
    AssertionError above ``atol + rtol``."""
    m = local_matrix(tile, direction)
    err = 0.0
    for t in range(tile):
        e = np.zeros(tile, dtype=np.complex128)
        e[t] = 1.0
        err = max(err, float(np.abs(m[:, t] - _local_stages(e, tile, direction)).max()))
    if err > atol + rtol:
        raise AssertionError(f"local matrix {direction} tile={tile}: err={err:.3e}")
    return err


def _global_stages(v: np.ndarray, from_log: int, to_log: int, direction: str) -> np.ndarray:
    """Stages of half-span 2^s, s in [from_log, to_log), over the whole
    array with the N-dependent twiddle exp(-2 pi i j N/(2 half) / N)
    (ascending for DIT, descending for DIF)."""
    n = v.size
    logs = list(range(from_log, to_log))
    for s in logs if direction == "dit" else logs[::-1]:
        h = 1 << s
        idx = np.arange(n).reshape(-1, 2 * h)
        j = np.arange(h)
        w = np.exp(-2j * np.pi * (j * (n // (2 * h))) / n)
        a, b = v[idx[:, :h]], v[idx[:, h:]]
        out = np.empty_like(v)
        if direction == "dit":
            out[idx[:, :h]], out[idx[:, h:]] = a + w * b, a - w * b
        else:
            out[idx[:, :h]], out[idx[:, h:]] = a + b, (a - b) * w
        v = out
    return v


def _blockwise(v: np.ndarray, m: np.ndarray) -> np.ndarray:
    t = m.shape[0]
    return (v.reshape(-1, t) @ m.T).reshape(-1)


def verify_decomposition(n: int, tile: int, direction: str = "dit", rtol=1e-10) -> float:
    """The local group composed with the remaining global stages gives the
    N-point DFT (``np.fft.fft``): DIT bit-reversed input -> local group ->
    global stages; DIF global stages -> local group -> bit-reversed output.
    A tile above ``n`` runs as ``tile = n``.  Returns the peak-relative
    error; AssertionError above ``rtol``."""
    logn = _log2_exact(n)
    tile = min(tile, n)
    logt = _log2_exact(tile)
    if n % tile:
        raise ValueError(f"tile={tile} must divide n={n}")
    rng = np.random.default_rng(1000003 * n + tile)
    x = rng.standard_normal(n) + 1j * rng.standard_normal(n)
    m = local_matrix(tile, direction)
    br = _bitrev(n)
    if direction == "dit":
        got = _global_stages(_blockwise(x[br], m), logt, logn, "dit")
    else:
        got = _blockwise(_global_stages(x, logt, logn, "dif"), m)[br]
    ref = np.fft.fft(x)
    rel = float(np.abs(got - ref).max()) / (float(np.abs(ref).max()) + 1.0)
    if rel > rtol:
        raise AssertionError(f"decomposition {direction} n={n} tile={tile}: rel={rel:.3e}")
    return rel


def _group_halves(n0: int, glog: int, direction: str) -> list:
    halves = [n0 << s for s in range(glog)]
    return halves if direction == "dit" else halves[::-1]


def tail_group_table(n0: int, glog: int, direction: str) -> np.ndarray:
    """complex128 ``[2^glog, P]`` table (``P = n0 << glog``) of one group
    of ``glog`` global stages starting at half-span ``n0``:
    ``out[i] = sum_k table[k, i mod P] * in[i ^ (k * n0)]``.  The stage
    twiddles exp(-2 pi i j / (2 half)) do not depend on N, so neither does
    the table."""
    if glog < 1:
        raise ValueError(f"glog must be >= 1, got {glog}")
    _log2_exact(n0)
    _direction(direction)
    p = n0 << glog
    g = np.eye(p, dtype=np.complex128)
    for h in _group_halves(n0, glog, direction):
        g = _stage(g, h, direction)  # rows are positions: the stage acts on every column
    i = np.arange(p)
    return np.stack([g[i, i ^ (k * n0)] for k in range(1 << glog)])


def tail_group_planar(n0: int, glog: int, direction: str):
    """``(C_r, C_i)`` float32, C-contiguous, of :func:`tail_group_table`."""
    t = tail_group_table(n0, glog, direction)
    return np.ascontiguousarray(t.real, dtype=np.float32), np.ascontiguousarray(t.imag, dtype=np.float32)


def apply_tail_group_table(v: np.ndarray, n0: int, glog: int, direction: str) -> np.ndarray:
    """The group applied through its table to every period-P block of ``v``."""
    t = tail_group_table(n0, glog, direction)
    p = t.shape[1]
    blocks = np.asarray(v).reshape(-1, p)
    i = np.arange(p)
    out = np.zeros_like(blocks, dtype=np.complex128)
    for k in range(t.shape[0]):
        out += t[k] * blocks[:, i ^ (k * n0)]
    return out.reshape(-1)


def verify_tail_group(n0: int, glog: int, direction: str, rtol: float = 1e-10) -> float:
    """The table against the group's stages applied one pair at a time, on
    random period vectors; peak-relative error, AssertionError above rtol."""
    p = n0 << glog
    rng = np.random.default_rng(7919 * p + glog + (direction == "dif"))
    err, scale = 0.0, 1.0
    for _ in range(4):
        v = rng.standard_normal(p) + 1j * rng.standard_normal(p)
        ref = v.copy()
        for h in _group_halves(n0, glog, direction):
            ref = _stage(ref, h, direction)
        err = max(err, float(np.abs(apply_tail_group_table(v, n0, glog, direction) - ref).max()))
        scale = max(scale, float(np.abs(v).max()) + 1.0)
    if err / scale > rtol:
        raise AssertionError(f"tail group {direction} n0={n0} glog={glog}: err={err:.3e}")
    return err / scale


def verify_grouped_decomposition(n: int, tile: int, glog: int, direction: str, rtol: float = 1e-10) -> float:
    """``n = tile << glog``: local group and one tail group (with the
    bit-reversal edges) give ``np.fft.fft``; peak-relative error."""
    if n != (tile << glog):
        raise ValueError(f"this check needs n == tile << glog, got n={n} tile={tile} glog={glog}")
    rng = np.random.default_rng(104729 * n + glog)
    x = rng.standard_normal(n) + 1j * rng.standard_normal(n)
    m = local_matrix(tile, direction)
    br = _bitrev(n)
    if direction == "dit":
        got = apply_tail_group_table(_blockwise(x[br], m), tile, glog, "dit")
    else:
        got = _blockwise(apply_tail_group_table(x, tile, glog, "dif"), m)[br]
    ref = np.fft.fft(x)
    rel = float(np.abs(got - ref).max()) / (float(np.abs(ref).max()) + 1.0)
    if rel > rtol:
        raise AssertionError(f"grouped decomposition {direction} n={n} tile={tile} glog={glog}: rel={rel:.3e}")
    return rel


def tail_groups(tile: int, logn: int, glog: int, maxp: int):
    """Partition the tail stages (half-spans ``tile .. 2^(logn-1)``,
    ascending) into ``(groups, singles)``: walking up from the smallest,
    each stage starts a group of the most stages ``s`` in ``[2, glog]``
    (and no more than remain) whose period ``n0 << s`` is at most ``maxp``;
    a stage that cannot start a group of two is a single.  ``groups`` is
    ``[(n0, s), ...]`` ascending, ``singles`` the half-spans left over."""
    if glog < 1:
        raise ValueError(f"glog must be >= 1, got {glog}")
    stages = [1 << s for s in range(_log2_exact(tile), logn)]
    groups, singles = [], []
    pos = 0
    while pos < len(stages):
        n0 = stages[pos]
        fits = [s for s in range(2, min(glog, len(stages) - pos) + 1) if (n0 << s) <= maxp]
        if fits:
            groups.append((n0, max(fits)))
            pos += max(fits)
        else:
            singles.append(n0)
            pos += 1
    return groups, singles
