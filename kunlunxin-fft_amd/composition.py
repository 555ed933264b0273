"""Exact-shape composition registry (reference src/xpu/composition.py).

On the P800 the registry promoted one vendor-core 4-step composition
(N=2048, B=16).  Here a composition is a four-step whose sub-FFT stages run
on a processing unit of the external-core registry (config/
external_cores.json): rocFFT through torch.fft ("vendor"), or this library's
own four-step ("local"); ``hybrid.run_hybrid`` executes it.
``composition_builder.py`` measures candidate compositions against the
selector's plan for exact shapes and writes config/composition_table.json,
which holds only entries past the 2% guard (its measurements travel with it).
The lookup fails closed: None unless a valid, profile- and environment-bound
table has an entry for the exact shape and the c2c forward/backward
semantic.
"""
from __future__ import annotations

import json
import os

from .config import CONFIG_DIR, ConfigError

TABLE_PATH = os.path.join(CONFIG_DIR, "composition_table.json")
KIND = "composition-promotion"
TABLE_REQUIRED_KEYS = ("kind", "profile_hash", "env_hash", "precision", "guard_pct", "entries")
ENTRY_REQUIRED_KEYS = ("N", "batch", "direction", "flow_id", "flow_realization",
                       "processing_unit", "candidate_ms", "incumbent_ms", "guard_pct", "reason", "tile", "core",
                       "evidence")
# what the builder measured for the entry: the plan it beat, every candidate's
# time, and the winner's relative L2 distance from the plan's output
EVIDENCE_REQUIRED_KEYS = ("incumbent", "candidates", "err_rel_l2")
MAX_ERR_REL_L2 = 1e-5


def guard_pct_of(candidate_ms: float, incumbent_ms: float) -> float:
    """Percent by which the candidate beats the incumbent (positive = faster)."""
    return (incumbent_ms - candidate_ms) / incumbent_ms * 100.0


def composition_entry_violations(entry: dict, table: dict) -> list[str]:
    """Contract violations of one composition entry (reference
    composition.py:64-114, on this library's entry fields): every required
    key; the DIT decomposition; a positive integer N and batch; a known
    core; a power-of-two tile of at least 16 dividing N; the stamped guard
    equal to the one its two medians give, and at least the table's; and
    the evidence, whose error is within the parity bound."""
    bad = [f"missing {k!r}" for k in ENTRY_REQUIRED_KEYS if entry.get(k) in (None, "")]
    if bad:
        return bad
    n, b, tile = entry["N"], entry["batch"], entry["tile"]
    if entry["direction"] != "dit":
        bad.append(f"direction {entry['direction']!r} (the composition is DIT only)")
    if not isinstance(n, int) or n <= 0:
        bad.append(f"N {n!r} not a positive int (exact keys only)")
    if not isinstance(b, int) or b <= 0:
        bad.append(f"batch {b!r} not a positive int")
    if entry["core"] not in ("vendor", "local", "triton"):
        bad.append(f"unknown core {entry['core']!r}")
    if not isinstance(tile, int) or tile < 16 or tile & (tile - 1) or (isinstance(n, int) and n % tile):
        bad.append(f"tile {tile!r} invalid (a power of two >= 16 dividing N)")
    g = guard_pct_of(float(entry["candidate_ms"]), float(entry["incumbent_ms"]))
    if abs(g - float(entry["guard_pct"])) > 1e-6:
        bad.append(f"guard_pct {entry['guard_pct']!r} != {g:.6f} recomputed from its medians")
    if g < float(table.get("guard_pct", 2.0)):
        bad.append(f"guard {g:.3f}% below {table.get('guard_pct')}%")
    ev = entry["evidence"]
    if not isinstance(ev, dict):
        return bad + ["evidence not an object"]
    bad += [f"evidence missing {k!r}" for k in EVIDENCE_REQUIRED_KEYS if ev.get(k) in (None, "")]
    err = ev.get("err_rel_l2")
    if isinstance(err, (int, float)) and not err <= MAX_ERR_REL_L2:
        bad.append(f"evidence err_rel_l2 {err} > {MAX_ERR_REL_L2} (parity gate)")
    return bad


def table_violations(table: dict) -> list[str]:
    bad = [f"missing table key {k!r}" for k in TABLE_REQUIRED_KEYS if table.get(k) in (None, "")]
    if bad:
        return bad
    if table["kind"] != KIND:
        bad.append(f"kind {table['kind']!r} != {KIND!r}")
    if not isinstance(table["entries"], list):
        return bad + ["entries not a list"]
    seen = set()
    for i, e in enumerate(table["entries"]):
        if not isinstance(e, dict):
            bad.append(f"entry {i} not an object")
            continue
        key = (e.get("N"), e.get("batch"), e.get("direction"))
        if key in seen:
            bad.append(f"duplicate exact-shape key {key}")
        seen.add(key)
        bad.extend(f"entry {key}: {msg}" for msg in composition_entry_violations(e, table))
    return bad


def load_composition_table(path: str = TABLE_PATH):
    """None when no table exists; ConfigError when one exists but is invalid."""
    try:
        with open(path) as f:
            table = json.load(f)
    except FileNotFoundError:
        return None
    except json.JSONDecodeError as e:
        raise ConfigError(f"composition table unreadable: {path}: {e}") from None
    if not isinstance(table, dict):
        raise ConfigError(f"composition table is not an object: {path}")
    v = table_violations(table)
    if v:
        raise ConfigError("composition table violates its contract: " + "; ".join(v[:8]))
    return table


_DEFAULT: dict = {}  # path -> ((mtime_ns, size), table or None) for plan-time lookups


def _default_composition_table(path: str = TABLE_PATH):
    """load_composition_table(path), re-read only when the file's modification
    time or size changes (planning queries it on every call); the returned
    dict is shared and is only read."""
    try:
        st = os.stat(path)
    except OSError:
        return load_composition_table(path)  # None, or the loader's error
    stamp = (st.st_mtime_ns, st.st_size)
    hit = _DEFAULT.get(path)
    if hit is not None and hit[0] == stamp:
        return hit[1]
    table = load_composition_table(path)
    _DEFAULT[path] = (stamp, table)
    return table


CORES_PATH = os.path.join(CONFIG_DIR, "external_cores.json")
EXTERNAL_CORES_PATH = CORES_PATH  # the reference's name
CLASSIFICATIONS = ("local-core", "materialized-external-subtransform", "full-transform-only", "boundary",
                   "reference-only", "unavailable")
CORE_REQUIRED_KEYS = ("id", "source", "api", "classification", "device_resident", "selector_status")


def load_external_cores(path: str = CORES_PATH) -> dict:
    """The processing-unit registry (reference config/external_cores.json),
    validated; ConfigError on a malformed registry."""
    try:
        with open(path) as f:
            reg = json.load(f)
    except (OSError, json.JSONDecodeError) as e:
        raise ConfigError(f"external-core registry unreadable: {path}: {e}") from None
    cores = reg.get("cores") if isinstance(reg, dict) else None
    if not isinstance(cores, list) or not cores:
        raise ConfigError("external-core registry: 'cores' must be a non-empty list")
    seen = set()
    for c in cores:
        miss = [k for k in CORE_REQUIRED_KEYS if c.get(k) in (None, "")]
        if miss:
            raise ConfigError(f"external-core registry: core {c.get('id')!r} misses {miss}")
        if c["classification"] not in CLASSIFICATIONS:
            raise ConfigError(f"external-core registry: {c['id']}: classification {c['classification']!r} "
                              f"not in {CLASSIFICATIONS}")
        if c["id"] in seen:
            raise ConfigError(f"external-core registry: duplicate id {c['id']!r}")
        seen.add(c["id"])
    return reg


def composition_cores(reg: dict | None = None) -> dict:
    """composition core name (HybridPlan.core) -> registry entry, for the
    cores a composition may use for its sub-FFT stages."""
    reg = reg if reg is not None else load_external_cores()
    return {c["composition_core"]: c for c in reg["cores"]
            if c.get("composition_core") and c["classification"] in ("local-core",
                                                                    "materialized-external-subtransform")}


def composition_select(direction: str, n: int, batch: int = 1, precision: str = "fp32",
                       profile_hash: str | None = None, env_hash: str | None = "auto",
                       table: dict | None = None, transform_type: str = "c2c",
                       transform_direction: str = "forward",
                       normalization: str = "backward"):
    """Exact-shape composition entry, or None (fail closed on any mismatch)."""
    if direction != "dit":
        return None
    if (transform_type, transform_direction, normalization) != ("c2c", "forward", "backward"):
        return None
    if table is None:
        table = _default_composition_table()
        if table is None:
            return None
    if precision != table.get("precision"):
        return None
    if not profile_hash or profile_hash != table.get("profile_hash"):
        return None
    bound = table.get("env_hash") or ""
    if not bound:
        return None
    if env_hash == "auto":
        from .envcheck import current_env_hash

        env_hash = current_env_hash()
    if env_hash is None or env_hash != bound:
        return None
    for e in table.get("entries", ()):
        if (e["N"], e["batch"], e["direction"]) == (n, batch, direction):
            return e
    return None
