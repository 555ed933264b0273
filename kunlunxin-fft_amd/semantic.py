"""Which flow ids a table entry of one transform type may name, and the
matrix semantics (reference src/xpu/semantic.py).

``plan_fft`` checks a selected entry's ``real_flow`` with
:func:`family_allows` before building the plan (the reference gates table
entries the same way, src/xpu/semantic.py:103-125).  The flow ids are this
build's: every transform type runs on the shared complex cores, and each
dedicated real flow belongs to its own transform type only.
"""
from __future__ import annotations

from dataclasses import dataclass

from .config import NORMALIZATIONS, TRANSFORM_DIRECTIONS, TRANSFORM_TYPES

# matrix label -> (transform_type, transform_direction, normalization): the
# four semantics of the reference's release matrix (semantic.py:36-43)
SEMANTIC_SPECS = {
    "c2c-forward": ("c2c", "forward", "backward"),
    "c2c-inverse": ("c2c", "inverse", "backward"),
    "r2c": ("r2c", "forward", "backward"),
    "c2r": ("c2r", "inverse", "backward"),
}

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


SPECIALIZED_FLOWS = REAL_FLOWS  # the reference's name (semantic.py:54-58)


@dataclass(frozen=True)
class SemanticSpec:
    label: str
    transform_type: str
    transform_direction: str
    normalization: str

    @property
    def key(self) -> tuple:
        """The selector's exact semantic key."""
        return (self.transform_type, self.transform_direction, self.normalization)


def spec(label: str) -> SemanticSpec:
    """The spec of one matrix label; KeyError for an unknown one."""
    if label not in SEMANTIC_SPECS:
        raise KeyError(f"unknown semantic label {label!r}; known: {sorted(SEMANTIC_SPECS)}")
    return SemanticSpec(label, *SEMANTIC_SPECS[label])


def family(transform_type: str) -> frozenset:
    """Every flow id an entry of ``transform_type`` may name."""
    if transform_type not in TRANSFORM_TYPES:
        raise KeyError(f"unknown transform_type {transform_type!r}; known: {TRANSFORM_TYPES}")
    return CORE_FLOWS | REAL_FLOWS[transform_type]


def family_allows(transform_type: str, flow_id: str) -> bool:
    """True when an entry of ``transform_type`` may name ``flow_id``."""
    return flow_id in family(transform_type)


def family_size(transform_type: str) -> int:
    return len(family(transform_type))


def validate_taxonomy() -> list[str]:
    """The specs and flow families agree with the key taxonomy (empty when
    they do)."""
    bad = []
    for label, (tt, td, norm) in SEMANTIC_SPECS.items():
        if tt not in TRANSFORM_TYPES:
            bad.append(f"{label}: transform_type {tt!r} not in the taxonomy")
        if td not in TRANSFORM_DIRECTIONS:
            bad.append(f"{label}: transform_direction {td!r} not in the taxonomy")
        if norm not in NORMALIZATIONS:
            bad.append(f"{label}: normalization {norm!r} not in the taxonomy")
    bad += [f"REAL_FLOWS missing {tt!r}" for tt in TRANSFORM_TYPES if tt not in REAL_FLOWS]
    return bad
