"""Frozen, measured per-shape selector (host-only: no torch import).

Contract kept from the reference (src/xpu/selector.py:1-41):

* **Key**: ``(profile_hash, env_hash, precision)`` for the whole table, then
  ``(N, batch, direction)`` plus the optional semantic triple
  ``(transform_type, transform_direction, normalization)`` per entry.
* **Tiers** (``find_entry``, selector.py:357-390): a ``previous_fallbacks``
  cell first, then an entry carrying the exact semantic triple, then a
  legacy entry without a triple (answers any semantic), else abstain.
* **Gates** (``select``, selector.py:524-646): bad semantic fields, a
  precision the table was not measured in, ``profile_hash`` missing or
  different, a table without ``env_hash``, an unknown live environment, or a
  different one -> ``source="abstain"`` with a reason; the caller then runs
  M0.  Nothing raises at lookup time.
* **Load-time contract** (``load_table``, selector.py:424-479): every entry's
  parameters must come from ``config/butterfly_space.json`` and name a runner
  of its own kernel family; a violating table is refused with ``ConfigError``.
* **M0 closure**: a challenger enters the table only if it beat the M0
  incumbent by ``GUARD_PCT`` percent (the builder, ``table_builder.py``).

The kernel families are MI355X ones: the reference's global-stage radix-2 /
radix-4 flows, plus the LDS-resident single-pass and four-step flows; the
reference's fused-inplace / matrix-resident / grouped-boundary families are
still accepted (their runner names run on the LDS kernels, see runner.py).
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field

from .config import (
    CONFIG_DIR,
    NORMALIZATIONS,
    TRANSFORM_DIRECTIONS,
    TRANSFORM_TYPES,
    ConfigError,
)

TABLE_PATH = os.path.join(CONFIG_DIR, "selector_table.json")

# Promotion guard in percent (reference selector.py:59-63).
GUARD_PCT = 2.0

# (flow_realization, processing_unit) -> legal runner names, per batch tier.
SINGLE_RUNNERS = {
    ("global-stage", "radix2-scalar"): frozenset({"fft_dit", "fft_dif"}),
    ("global-stage", "radix4-scalar"): frozenset({"fft_dit_radix4", "fft_dif_radix4"}),
    ("lds-resident", "stockham-radix16"): frozenset({"fft_lds_fused"}),
    ("four-step", "stockham-radix16"): frozenset({"fft_four_step"}),
    ("matrix-resident", "dense-dot-fft64"): frozenset({"fft_dit_matrix", "fft_dif_matrix"}),
    ("fused-inplace", "radix2-scalar"): frozenset({"fft_dit_fused"}),
    ("grouped-boundary", "composite-linear-map"): frozenset({"fft_dit_grouped", "fft_dif_grouped"}),
}
BATCH_RUNNERS = {
    ("global-stage", "radix2-scalar"): frozenset({"fft_dit_batch", "fft_dif_batch"}),
    ("global-stage", "radix4-scalar"): frozenset({"fft_dit_radix4_batch", "fft_dif_radix4_batch"}),
    ("lds-resident", "stockham-radix16"): frozenset({"fft_lds_fused_batch"}),
    ("four-step", "stockham-radix16"): frozenset({"fft_four_step_batch"}),
    ("matrix-resident", "dense-dot-fft64"): frozenset({"fft_dit_matrix_batch", "fft_dif_matrix_batch"}),
}

# Per-cell fallback binding (reference selector.py:260-340).
FALLBACK_CARRY_CONTRACT = "fallback-env-binding-v1"
FALLBACK_BINDING_KEYS = ("carry_contract", "source_env_hash", "source_profile_hash",
                         "source_precision", "source_device", "source_table_sha256",
                         "source_result_sha256", "paired_confirm")
DEVICE_IDENTITY_KEYS = ("device_model", "multiprocessor_count", "max_shared_mem")


def _is_pow2(v) -> bool:
    return isinstance(v, int) and v > 0 and (v & (v - 1)) == 0


def entry_contract_violations(entry: dict, space=None) -> list[str]:
    """Design-space and runner-family violations of one table entry
    (``space``: the loaded DesignSpace, read from disk when None)."""
    from .config import DesignSpace

    sp = space
    if sp is None:
        try:
            sp = DesignSpace.load()
        except ConfigError as e:
            return [f"design space unreadable: {e}"]
    bad: list[str] = []
    n, batch = entry.get("N"), entry.get("batch")
    if not _is_pow2(n):
        bad.append(f"N {n!r} not a positive power of two")
    if not isinstance(batch, int) or batch < 1:
        bad.append(f"batch {batch!r} not a positive int")
    if entry.get("direction") not in ("dit", "dif"):
        bad.append(f"direction {entry.get('direction')!r} not dit/dif")
    block = entry.get("block")
    if not _is_pow2(block):
        bad.append(f"block {block!r} not a positive power of two")
    params = dict(entry.get("params") or {})
    real, unit = entry.get("flow_realization"), entry.get("processing_unit")
    fam = (real, unit)
    if fam not in SINGLE_RUNNERS:
        bad.append(f"unknown kernel family (flow_realization={real!r}, processing_unit={unit!r})")
    if unit == "radix4-scalar" and 4 not in sp.radix:
        bad.append("radix-4 not in the published radix space")
    if real == "global-stage" and isinstance(block, int) and block not in sp.stage_blocks:
        bad.append(f"block {block} not in global-stage blocks {sp.stage_blocks}")
    if real == "lds-resident":
        e = params.get("elems", 0)
        if e not in (0,) + sp.lds_elems:
            bad.append(f"elems {e!r} not in {sp.lds_elems}")
        stg = params.get("stagger", 0)
        if stg not in (0,) + sp.lds_stagger:
            bad.append(f"stagger {stg!r} not in {sp.lds_stagger}")
        stage = params.get("stage", 0)
        if stage not in (0,) + sp.lds_staged:
            bad.append(f"stage {stage!r} not in {sp.lds_staged}")
        if isinstance(n, int) and n > 2 * sp.lds_max_n:
            bad.append(f"N={n} exceeds the LDS kernel's range ({sp.lds_max_n} complex core)")
    if real == "matrix-resident":
        if params.get("elems") or params.get("n1") or params.get("stagger"):
            bad.append("the dense-dot matrix-core flow takes no elems / stagger / n1 parameters")
        if isinstance(n, int) and n > 2 * sp.dense_max_n:
            bad.append(f"N={n} exceeds the dense-dot core's range ({sp.dense_max_n} complex core)")
    if real == "four-step":
        n1 = params.get("n1", 0)
        if n1 not in (0,) + sp.fourstep_n1:
            bad.append(f"n1 {n1!r} not in {sp.fourstep_n1}")
        ch = params.get("chunk_rows", 0)
        if ch not in sp.fourstep_chunk_rows:
            bad.append(f"chunk_rows {ch!r} not in {sp.fourstep_chunk_rows}")
        sched = params.get("schedule", 0)
        if sched not in sp.fourstep_schedule:
            bad.append(f"schedule {sched!r} not in {sp.fourstep_schedule}")
        order = params.get("pass2_order", 0)
        if order not in sp.fourstep_pass2_order:
            bad.append(f"pass2_order {order!r} not in {sp.fourstep_pass2_order}")
        if isinstance(n, int) and n < sp.fourstep_min_n:
            bad.append(f"N={n} below the four-step minimum {sp.fourstep_min_n}")
    if "variant" in params and params["variant"] not in sp.batch_variants:
        bad.append(f"variant {params['variant']!r} not in {sp.batch_variants}")
    if "transform_type" in entry:
        if entry.get("transform_type") not in TRANSFORM_TYPES:
            bad.append(f"transform_type {entry.get('transform_type')!r} not in {TRANSFORM_TYPES}")
        if entry.get("transform_direction") not in TRANSFORM_DIRECTIONS:
            bad.append(f"transform_direction {entry.get('transform_direction')!r} not in {TRANSFORM_DIRECTIONS}")
        if entry.get("normalization") not in NORMALIZATIONS:
            bad.append(f"normalization {entry.get('normalization')!r} not in {NORMALIZATIONS}")
    executed = entry.get("executed")
    if executed is not None and fam in SINGLE_RUNNERS:
        b = int(params.get("batch") or batch or 1) if isinstance(batch, int) else 1
        allowed = (BATCH_RUNNERS if b > 1 else SINGLE_RUNNERS).get(fam, frozenset())
        if executed not in allowed:
            bad.append(f"executed {executed!r} not a legal runner of {fam} at batch={b} "
                       f"(allowed: {sorted(allowed)})")
    return bad


def semantic_key_of(entry: dict):
    """Exact semantic triple of an entry, or None for a legacy entry."""
    if "transform_type" not in entry:
        return None
    return (entry.get("transform_type"), entry.get("transform_direction"), entry.get("normalization"))


def fallback_binding_violations(table: dict) -> list[str]:
    """Every previous_fallbacks cell must be bound to this table's
    environment, profile, precision and device (reference selector.py:279-340)."""
    out: list[str] = []
    ident = {k: (table.get("env") or {}).get(k) for k in DEVICE_IDENTITY_KEYS}
    for i, e in enumerate(table.get("previous_fallbacks") or ()):
        key = (e.get("N"), e.get("batch"), e.get("direction"))
        prov = e.get("previous_fallback_provenance")
        if not isinstance(prov, dict):
            out.append(f"previous_fallbacks[{i}] {key}: missing previous_fallback_provenance")
            continue
        missing = [k for k in FALLBACK_BINDING_KEYS if prov.get(k) in (None, "")]
        if missing:
            out.append(f"previous_fallbacks[{i}] {key}: provenance missing binding key(s) {', '.join(missing)}")
            continue
        if prov["carry_contract"] != FALLBACK_CARRY_CONTRACT:
            out.append(f"previous_fallbacks[{i}] {key}: carry_contract {prov['carry_contract']!r}")
        if prov["source_env_hash"] != table.get("env_hash"):
            out.append(f"previous_fallbacks[{i}] {key}: source env {prov['source_env_hash']} != "
                       f"table env {table.get('env_hash')}")
        if prov["source_profile_hash"] != table.get("profile_hash"):
            out.append(f"previous_fallbacks[{i}] {key}: source profile differs from the table's")
        if prov["source_precision"] != table.get("precision"):
            out.append(f"previous_fallbacks[{i}] {key}: source precision differs from the table's")
        if any(v is None for v in ident.values()):
            out.append(f"previous_fallbacks[{i}] {key}: table carries no device identity")
        elif prov["source_device"] != ident:
            out.append(f"previous_fallbacks[{i}] {key}: source device {prov['source_device']} != {ident}")
    return out


def is_previous_fallback(table: dict, entry: dict) -> bool:
    return any(entry is e for e in (table.get("previous_fallbacks") or ()))


def _cell_index(table: dict) -> tuple:
    """(fallbacks, entries, batches): the previous-fallback cells by (N,
    batch, direction, semantic key), first of each kept; the entries by (N,
    batch, direction), in table order; the sorted batches of the entries by
    (N, direction)."""
    fb, ent, bat = {}, {}, {}
    for e in table.get("previous_fallbacks") or ():
        fb.setdefault((e["N"], e["batch"], e["direction"], semantic_key_of(e)), e)
    for e in table.get("entries", ()):
        ent.setdefault((e["N"], e["batch"], e["direction"]), []).append(e)
        bat.setdefault((e["N"], e["direction"]), set()).add(e["batch"])
    return fb, ent, {k: sorted(v) for k, v in bat.items()}


def _table_batches(table: dict, n: int, direction: str) -> list:
    """Sorted batches the table holds entries for at (N, direction)."""
    idx = _INDEX.get(id(table))
    if idx is not None and idx[0] is table:
        return idx[1][2].get((n, direction), [])
    return sorted({e["batch"] for e in table.get("entries", ()) if (e["N"], e["direction"]) == (n, direction)})


def rounded_batch(table: dict, n: int, batch: int, direction: str, transform_type: str = "c2c",
                  transform_direction: str = "forward", normalization: str = "backward"):
    """The table batch whose measured decision a batch with no exact key
    takes: the smallest table batch at or above it (the next power of two,
    on a grid of powers of two), or past the table's largest batch of this N
    that largest one; None when no batch of this N, direction and semantic
    has an entry."""
    sem = (transform_type, transform_direction, normalization)
    # batched entries only for a batch above 1 (their runners are the batch forms)
    have = [b for b in _table_batches(table, n, direction)
            if (b > 1 or batch == 1) and find_entry(table, n, b, direction, *sem) is not None]
    if not have:
        return None
    above = [b for b in have if b >= batch]
    return above[0] if above else have[-1]


def find_entry(table: dict, n: int, batch: int, direction: str, transform_type: str = "c2c",
               transform_direction: str = "forward", normalization: str = "backward"):
    """previous-fallback cell > exact semantic entry > legacy entry > None."""
    want = (transform_type, transform_direction, normalization)
    idx = _INDEX.get(id(table))
    if idx is not None and idx[0] is table:
        # the package's shared table (default_table): indexed once per file
        # version, the same answer as the scan below
        fb, ent = idx[1][0], idx[1][1]
        hit = fb.get((n, batch, direction, want))
        if hit is not None:
            return hit
        legacy = None
        for e in ent.get((n, batch, direction), ()):
            sk = semantic_key_of(e)
            if sk == want:
                return e
            if sk is None and legacy is None:
                legacy = e
        return legacy
    for e in table.get("previous_fallbacks") or ():
        if (e["N"], e["batch"], e["direction"]) == (n, batch, direction) and semantic_key_of(e) == want:
            return e
    legacy = None
    for e in table.get("entries", ()):
        if (e["N"], e["batch"], e["direction"]) != (n, batch, direction):
            continue
        sk = semantic_key_of(e)
        if sk == want:
            return e
        if sk is None and legacy is None:
            legacy = e
    return legacy


@dataclass(frozen=True)
class Selection:
    """One selector verdict; ``source`` is ``"table"`` or ``"abstain"``."""

    n: int
    direction: str
    batch: int
    precision: str
    source: str
    reason: str
    transform_type: str = "c2c"
    transform_direction: str = "forward"
    normalization: str = "backward"
    entry_tier: str = "abstain"
    block: int | None = None
    flow_id: str | None = None
    flow_realization: str | None = None
    processing_unit: str | None = None
    params: dict = field(default_factory=dict)
    incumbent_ms: float | None = None
    challenger_ms: float | None = None
    executed: str | None = None
    table_batch: int | None = None  # entry tier batch-rounded: the table batch whose decision applies

    @property
    def selected(self) -> bool:
        return self.source == "table"


def load_table(path: str = TABLE_PATH) -> dict:
    """Load and contract-check a selector table (ConfigError on any violation)."""
    try:
        with open(path) as f:
            table = json.load(f)
    except FileNotFoundError:
        raise ConfigError(f"selector table not found: {path}") from None
    except json.JSONDecodeError as e:
        raise ConfigError(f"selector table unreadable: {path}: {e}") from None
    if not isinstance(table, dict):
        raise ConfigError(f"selector table is not an object: {path}")
    for key in ("profile_hash", "precision", "guard_pct", "entries"):
        if key not in table:
            raise ConfigError(f"selector table missing required key {key!r}")
    from .config import DesignSpace

    try:
        space = DesignSpace.load()
    except ConfigError as e:
        raise ConfigError(f"selector table cannot be checked: design space unreadable: {e}") from None
    problems: list[str] = []
    for e in table["entries"]:
        key = (e.get("N"), e.get("batch"), e.get("direction"))
        problems += [f"entry {key}: {m}" for m in entry_contract_violations(e, space)]
    seen: set = set()
    for i, e in enumerate(table.get("previous_fallbacks") or []):
        key = (e.get("N"), e.get("batch"), e.get("direction"))
        sk = semantic_key_of(e)
        if sk is None:
            problems.append(f"previous_fallbacks[{i}] {key}: missing the exact semantic triple")
        elif key + sk in seen:
            problems.append(f"previous_fallbacks[{i}] {key} {sk}: duplicate cell")
        else:
            seen.add(key + sk)
        problems += [f"previous_fallbacks[{i}] {key}: {m}" for m in entry_contract_violations(e, space)]
    problems += fallback_binding_violations(table)
    if problems:
        raise ConfigError(f"selector table violates the design space / runner contract "
                          f"({len(problems)}): " + "; ".join(problems[:8])
                          + (" ..." if len(problems) > 8 else ""))
    return table


_DEFAULT: dict = {}  # path -> ((mtime_ns, size), validated table) for plan-time lookups
_INDEX: dict = {}  # id(table) -> (table, _cell_index(table)) for the tables default_table shares


def default_table(path: str = TABLE_PATH) -> dict:
    """The package's table for plan-time lookups: ``load_table(path)``,
    re-read and re-checked only when the file's modification time or size
    changes.  The returned dict is shared and must not be modified (the
    planner copies what it keeps); ``load_table`` gives a private copy."""
    try:
        st = os.stat(path)
    except OSError:
        return load_table(path)  # raises the loader's error
    stamp = (st.st_mtime_ns, st.st_size)
    hit = _DEFAULT.get(path)
    if hit is not None and hit[0] == stamp:
        return hit[1]
    table = load_table(path)
    old = _DEFAULT.get(path)
    if old is not None:
        _INDEX.pop(id(old[1]), None)
    _DEFAULT[path] = (stamp, table)
    _INDEX[id(table)] = (table, _cell_index(table))
    return table


def assert_current_environment(table: dict) -> str:
    """Freshness gate for measurement runs (reference selector.py:482-510):
    raise ``RuntimeError`` unless the live environment fingerprint equals the
    table's ``env_hash``, before any kernel launch; a table without one, or
    an environment that cannot be fingerprinted, fails closed too.  Returns
    the live hash so a run can record it."""
    bound = table.get("env_hash") or ""
    if not bound:
        raise RuntimeError("selector table carries no env_hash; refusing to measure against it "
                           "-- rebuild the table under the current environment")
    from .envcheck import current_env_hash

    cur = current_env_hash()
    if cur is None:
        raise RuntimeError("live environment fingerprint unknown (no GPU, or the library is not built); "
                           "cannot verify the table -- failing closed")
    if cur != bound:
        raise RuntimeError(f"environment hash {cur} != table {bound} (device, runtime or library changed "
                           "since the table was built); re-measure before producing new results")
    return cur


def _abstain(n, direction, batch, precision, reason, tt, td, norm) -> Selection:
    return Selection(n=n, direction=direction, batch=batch, precision=precision, source="abstain",
                     reason=reason, transform_type=tt, transform_direction=td,
                     normalization=norm, entry_tier="abstain")


def select(direction: str, n: int, batch: int = 1, precision: str = "fp32",
           profile_hash: str | None = None, table: dict | None = None,
           env_hash: str | None = "auto", transform_type: str = "c2c",
           transform_direction: str = "forward", normalization: str = "backward") -> Selection:
    """Measured winner for one shape, or an abstain verdict with its reason."""
    table = table if table is not None else default_table()
    sem = (transform_type, transform_direction, normalization)

    def no(reason: str) -> Selection:
        return _abstain(n, direction, batch, precision, reason, *sem)

    if transform_type not in TRANSFORM_TYPES:
        return no(f"transform_type must be one of {TRANSFORM_TYPES}, got {transform_type!r}")
    if transform_direction not in TRANSFORM_DIRECTIONS:
        return no(f"transform_direction must be one of {TRANSFORM_DIRECTIONS}, got {transform_direction!r}")
    if normalization not in NORMALIZATIONS:
        return no(f"normalization must be one of {NORMALIZATIONS}, got {normalization!r}")
    if direction not in ("dit", "dif"):
        return no(f"direction must be dit/dif, got {direction!r}")
    if precision != table["precision"]:
        return no(f"table measured {table['precision']}, got {precision!r}")
    if profile_hash is None:
        return no("profile_hash is required; None cannot bypass the table (fall back to M0)")
    if profile_hash != table["profile_hash"]:
        return no(f"profile hash {profile_hash} != table {table['profile_hash']}; "
                  "re-measure before selecting")
    bound = table.get("env_hash") or ""
    if not bound:
        return no("table carries no env_hash (unbound table); runtime selection fails closed to M0")
    cur = env_hash
    if cur == "auto":
        from .envcheck import current_env_hash

        cur = current_env_hash()
    if cur is None:
        return no("environment fingerprint unknown (device/runtime not probeable); "
                  "this table cannot be verified here and fails closed to M0")
    if cur != bound:
        return no(f"environment hash {cur} != table {bound} (device/runtime changed since "
                  "the table was built); re-measure before selecting")
    e = find_entry(table, n, batch, direction, *sem)
    rounded = None
    if e is None and batch > 1:
        # no exact key (a batch that is not a power of two, or past the grid):
        # the measured decision of the nearest table batch of this N
        rounded = rounded_batch(table, n, batch, direction, *sem)
        if rounded is not None:
            e = find_entry(table, n, rounded, direction, *sem)
    if e is None:
        return no(f"no measured entry for N={n} batch={batch} direction={direction} "
                  f"semantic={transform_type}/{transform_direction}/{normalization}; fall back to M0")
    if is_previous_fallback(table, e):
        tier = "previous-fallback"
        reason = "previous-deployed per-cell fallback: " + e.get("reason", "measured confirmation winner")
    else:
        tier = "semantic" if semantic_key_of(e) is not None else "legacy"
        reason = e.get("reason", "measured confirmation winner")
    if rounded is not None:
        reason = (f"no entry for batch={batch}; the measured decision of batch={rounded} ({tier} entry) "
                  f"applies: {reason}")
        tier = "batch-rounded"
    return Selection(
        n=n, direction=direction, batch=batch, precision=precision, source="table", reason=reason,
        transform_type=transform_type, transform_direction=transform_direction,
        normalization=normalization, entry_tier=tier, block=e["block"], flow_id=e["flow_id"],
        flow_realization=e["flow_realization"], processing_unit=e["processing_unit"],
        params=dict(e.get("params") or {}), incumbent_ms=e.get("incumbent_ms"),
        challenger_ms=e.get("challenger_ms"), executed=e.get("executed"), table_batch=rounded,
    )
