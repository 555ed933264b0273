"""Phase hooks around execute_fft_plan (reference src/xpu/ledger.py:64-148).

``phase(name)`` is a shared no-op context unless a ``PhaseLedger`` is
active; an active ledger synchronises the device around each phase and
records its wall time.  Hardware evidence (bytes, bank conflicts) comes from
rocprofv3 counters, not from this ledger.
"""
from __future__ import annotations

import contextlib
import time

_active = None


class _Noop:
    __slots__ = ()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


_NOOP = _Noop()


class PhaseLedger:
    """Collects (phase, seconds) rows while active (``with PhaseLedger() as l:``)."""

    def __init__(self, sync: bool = True):
        self.sync = sync
        self.rows: list[tuple[str, float]] = []
        self._prev = None

    def __enter__(self):
        global _active
        self._prev, _active = _active, self
        return self

    def __exit__(self, *exc):
        global _active
        _active = self._prev
        return False

    def _sync(self):
        if self.sync:
            import torch

            if torch.cuda.is_available():
                torch.cuda.synchronize()

    @contextlib.contextmanager
    def measure(self, name: str):
        self._sync()
        t0 = time.perf_counter()
        try:
            yield
        finally:
            self._sync()
            self.rows.append((name, time.perf_counter() - t0))

    def totals(self) -> dict:
        out: dict = {}
        for name, s in self.rows:
            out[name] = out.get(name, 0.0) + s
        return out


def phase(name: str):
    """Context for one execute phase; free when no ledger is active."""
    if _active is None:
        return _NOOP
    return _active.measure(name)
