"""Which flow ids a table entry of one transform type may name.

``plan_fft`` checks a selected entry's ``real_flow`` with
:func:`family_allows` before building the plan (the reference gates table
entries the same way, src/xpu/semantic.py:103-125).  The flow ids are this
build's: every transform type runs on the shared complex cores, and each
dedicated real flow belongs to its own transform type only.
"""
from __future__ import annotations

from .config import TRANSFORM_TYPES

# complex cores every transform type may run on
CORE_FLOWS = frozenset({
    "baseline-global-stage",     # M0 radix-2 / M5 radix-4, one launch per stage
    "batch-folded",              # the same with the batch folded into the grid
    "local-fused-tile",          # reference M1/M2 name; the single-pass LDS kernel here
    "lds-stockham-single-pass",
    "four-step-two-pass",
})

# the half-length real flows, one per real transform type
REAL_FLOWS = {
    "c2c": frozenset(),
    "r2c": frozenset({"dedicated-r2c-pack-v1"}),
    "c2r": frozenset({"dedicated-c2r-hermitian-v1"}),
}


def family_allows(transform_type: str, flow_id: str) -> bool:
    """True when an entry of ``transform_type`` may name ``flow_id``."""
    if transform_type not in TRANSFORM_TYPES:
        raise KeyError(f"unknown transform_type {transform_type!r}; known: {TRANSFORM_TYPES}")
    return flow_id in CORE_FLOWS or flow_id in REAL_FLOWS[transform_type]
