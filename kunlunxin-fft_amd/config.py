"""Configuration loading (host-only: no torch import).

Mirrors the reference's ``src/xpu/config.py`` contract -- ``ConfigError``,
the semantic-key taxonomy, a ``DeviceProfile`` whose ``hash()`` binds a
selector table to a device, and a ``DesignSpace`` that every table entry's
parameters must come from -- with MI355X facts in place of the P800 ones.

* ``DeviceProfile.hash()`` is sha256 of the sorted-key JSON of the profile,
  first 16 hex digits (config.py:94-95 of the reference).
* ``SizeMatrix`` holds the correctness / bench length lists (reference
  config.py:98-125); ``Manifest`` / ``build_manifest`` / ``git_commit`` /
  ``git_dirty`` are the per-run provenance record (config.py:268-352).
* The JSON files live in this package's ``config/`` directory.
"""
from __future__ import annotations

import hashlib
import json
import os
import subprocess
from dataclasses import asdict, dataclass, field

_PKG = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_PKG)
CONFIG_DIR = os.path.join(_PKG, "config")


class ConfigError(ValueError):
    """Raised when a config file is missing, unreadable, or fails its schema
    (reference config.py:24-25)."""


# Semantic key taxonomy (reference config.py:34-36).
TRANSFORM_TYPES = ("c2c", "r2c", "c2r")
TRANSFORM_DIRECTIONS = ("forward", "inverse")
NORMALIZATIONS = ("none", "forward", "backward", "ortho")


def _read_json(name: str) -> dict:
    path = os.path.join(CONFIG_DIR, name)
    if not os.path.exists(path):
        raise ConfigError(f"missing config file: {path}")
    with open(path) as f:
        try:
            return json.load(f)
        except json.JSONDecodeError as e:
            raise ConfigError(f"{path} is not valid JSON: {e}") from e


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ConfigError(msg)


def _pow2_list(v) -> bool:
    return (isinstance(v, list) and bool(v)
            and all(isinstance(t, int) and t > 0 and (t & (t - 1)) == 0 for t in v))


@dataclass(frozen=True)
class DeviceProfile:
    """Validated MI355X hardware profile (config/device.json).

    Static facts only; the live runtime/driver binding is the separate
    environment fingerprint (``envcheck``), as in the reference.
    """

    device: str
    board: str
    gfx_arch: str
    compute_units: int
    xcds: int
    wavefront_size: int
    lds_bytes_per_cu: int
    hbm_gib: int
    hbm_peak_gbps: int
    device_code_path: str
    torch_device_key: str
    baseline: str
    max_n: int

    @staticmethod
    def load() -> "DeviceProfile":
        d = _read_json("device.json")
        for key in ("device", "board", "gfx_arch", "device_code_path", "torch_device_key", "baseline"):
            _require(isinstance(d.get(key), str) and d[key],
                     f"device.json: {key} must be a non-empty string")
        for key in ("compute_units", "xcds", "wavefront_size", "lds_bytes_per_cu", "hbm_gib",
                    "hbm_peak_gbps", "max_n"):
            _require(isinstance(d.get(key), int) and d[key] > 0,
                     f"device.json: {key} must be a positive int")
        return DeviceProfile(**{k: d[k] for k in DeviceProfile.__dataclass_fields__})

    def hash(self) -> str:
        return hashlib.sha256(json.dumps(asdict(self), sort_keys=True).encode()).hexdigest()[:16]


@dataclass(frozen=True)
class DesignSpace:
    """The published MI355X candidate space (config/butterfly_space.json).

    Every selector-table entry's parameters must be drawn from these lists;
    the table loader refuses a table that names anything else (reference
    selector.py:140-248 contract, rebuilt for the HIP kernels).
    """

    space_id: str
    target: str
    radix: tuple
    stage_blocks: tuple
    lds_elems: tuple
    lds_max_n: int
    lds_stagger: tuple
    lds_staged: tuple
    dense_max_n: int
    fourstep_n1: tuple
    fourstep_chunk_rows: tuple
    fourstep_min_n: int
    fourstep_schedule: tuple
    fourstep_pass2_order: tuple
    batch_candidates: tuple
    batch_variants: tuple
    layout_in: str
    layout_out: str

    @staticmethod
    def load() -> "DesignSpace":
        d = _read_json("butterfly_space.json")
        _require(isinstance(d.get("space_id"), str) and d["space_id"], "butterfly_space.json: space_id required")
        _require(isinstance(d.get("target"), str) and d["target"], "butterfly_space.json: target required")
        p = d.get("P", {})
        _require(_pow2_list(p.get("radix")), "butterfly_space.json: P.radix must be powers of two")
        st = p.get("global_stage", {})
        _require(_pow2_list(st.get("blocks")), "butterfly_space.json: P.global_stage.blocks must be powers of two")
        lds = p.get("lds_fused", {})
        dense = p.get("dense_mfma", {})
        _require(isinstance(dense.get("max_n"), int) and 2 <= dense["max_n"] <= 16384,
                 "butterfly_space.json: P.dense_mfma.max_n must be in [2, 16384]")
        _require(_pow2_list(lds.get("elems")), "butterfly_space.json: P.lds_fused.elems must be powers of two")
        _require(isinstance(lds.get("max_n"), int) and lds["max_n"] > 0, "butterfly_space.json: P.lds_fused.max_n required")
        stag = lds.get("stagger", [0])
        _require(isinstance(stag, list) and stag and all(isinstance(v, int) and 0 <= v <= 16 for v in stag),
                 "butterfly_space.json: P.lds_fused.stagger must be ints in [0, 16]")
        staged = lds.get("staged", [0])
        _require(isinstance(staged, list) and staged and all(v in (0, 1) for v in staged),
                 "butterfly_space.json: P.lds_fused.staged must be a list of 0 / 1")
        fs = p.get("four_step", {})
        _require(_pow2_list(fs.get("n1")), "butterfly_space.json: P.four_step.n1 must be powers of two")
        ch = fs.get("chunk_rows")
        _require(isinstance(ch, list) and ch and all(isinstance(c, int) and c >= 0 for c in ch),
                 "butterfly_space.json: P.four_step.chunk_rows must be non-negative ints")
        _require(isinstance(fs.get("min_n"), int) and fs["min_n"] > 0, "butterfly_space.json: P.four_step.min_n required")
        sched = fs.get("schedule", [0])
        _require(isinstance(sched, list) and sched and all(v in (0, 1, 2, 3) for v in sched),
                 "butterfly_space.json: P.four_step.schedule must be a list of 0/1/2/3")
        order = fs.get("pass2_order", [0])
        _require(isinstance(order, list) and order and all(v in (0, 1) for v in order),
                 "butterfly_space.json: P.four_step.pass2_order must be a list of 0/1")
        b = p.get("batch_expansion", {})
        _require(_pow2_list(b.get("candidates")), "butterfly_space.json: P.batch_expansion.candidates must be powers of two")
        variants = b.get("variants", [])
        _require(isinstance(variants, list) and all(v in ("spread", "folded") for v in variants),
                 "butterfly_space.json: P.batch_expansion.variants must be 'spread'/'folded'")
        lay = d.get("L", {})
        _require(isinstance(lay.get("in"), list) and lay["in"], "butterfly_space.json: L.in required")
        _require(isinstance(lay.get("out"), list) and lay["out"], "butterfly_space.json: L.out required")
        return DesignSpace(
            space_id=d["space_id"], target=d["target"], radix=tuple(p["radix"]),
            stage_blocks=tuple(st["blocks"]), lds_elems=tuple(lds["elems"]), lds_max_n=lds["max_n"],
            lds_stagger=tuple(stag), lds_staged=tuple(staged), dense_max_n=dense["max_n"],
            fourstep_n1=tuple(fs["n1"]), fourstep_chunk_rows=tuple(ch), fourstep_min_n=fs["min_n"],
            fourstep_schedule=tuple(sched), fourstep_pass2_order=tuple(order),
            batch_candidates=tuple(b["candidates"]), batch_variants=tuple(variants),
            layout_in=lay["in"][0], layout_out=lay["out"][0],
        )


@dataclass(frozen=True)
class SizeMatrix:
    """Validated length lists (config/sizes.json; reference config.py:98-125):
    the correctness and benchmark lengths, the global-stage workgroup sizes
    and the largest length the vendor comparison column runs at."""

    correctness_sizes: tuple
    bench_sizes: tuple
    blocksizes: tuple
    vendor_baseline_max_n: int

    @staticmethod
    def load() -> "SizeMatrix":
        d = _read_json("sizes.json")
        for key in ("correctness_sizes", "bench_sizes", "blocksizes"):
            v = d.get(key)
            _require(isinstance(v, list) and bool(v), f"sizes.json: {key} must be a non-empty list")
            _require(all(isinstance(t, int) and not isinstance(t, bool) and t > 0 for t in v),
                     f"sizes.json: {key} must be positive ints")
            _require(all((t & (t - 1)) == 0 for t in v), f"sizes.json: {key} must be powers of two")
        _require(isinstance(d.get("vendor_baseline_max_n"), int) and not isinstance(d["vendor_baseline_max_n"], bool),
                 "sizes.json: vendor_baseline_max_n must be an int")
        return SizeMatrix(correctness_sizes=tuple(d["correctness_sizes"]), bench_sizes=tuple(d["bench_sizes"]),
                          blocksizes=tuple(d["blocksizes"]), vendor_baseline_max_n=d["vendor_baseline_max_n"])


def git_commit() -> str:
    """Best-effort commit hash of the checkout this package sits in;
    ``"unknown"`` outside a git checkout."""
    try:
        out = subprocess.run(["git", "rev-parse", "HEAD"], cwd=_ROOT, capture_output=True, text=True, timeout=10)
        return out.stdout.strip() or "unknown"
    except (OSError, subprocess.SubprocessError):
        return "unknown"


def git_dirty() -> bool:
    """True when tracked files differ from HEAD (untracked run output is
    ignored: it cannot change the code a run executes); False outside a
    checkout."""
    try:
        out = subprocess.run(["git", "status", "--porcelain", "--untracked-files=no"], cwd=_ROOT,
                             capture_output=True, text=True, timeout=10)
        return out.returncode == 0 and bool(out.stdout.strip())
    except (OSError, subprocess.SubprocessError):
        return False


@dataclass
class Manifest:
    """Per-run provenance record (reference config.py:302-333), with the
    MI355X profile's fields: ``gfx_arch`` where the reference records its
    XPU architecture number, and ``env_hash`` for the live runtime/driver
    fingerprint (``envcheck``), which the reference keeps as ``driver``."""

    commit: str
    dirty: bool
    profile_hash: str
    device: str
    gfx_arch: str
    torch_device_key: str
    env_hash: str | None = None
    dtype: str = "complex64"
    direction: str = "forward"
    precision: str = "fp32"
    flow_id: str = "baseline-global-stage"
    processing_unit: str = "radix2-scalar"
    us: int = 1
    ts: int = 1
    ud: int = 1
    td: int = 1
    boundary_residence: str = "gm"
    layout: str = "interleaved-complex64"
    block: int = 256
    fused_tile: int = 1
    warmup: int = 10
    trials: int = 50
    correctness_threshold: float = 1e-4
    command: str = ""
    extra: dict = field(default_factory=dict)

    def to_dict(self) -> dict:
        return asdict(self)


def build_manifest(profile: DeviceProfile, **overrides) -> Manifest:
    """A manifest pinned to the current commit and ``profile``; keyword
    overrides must name existing fields (``ConfigError`` otherwise)."""
    m = Manifest(commit=git_commit(), dirty=git_dirty(), profile_hash=profile.hash(), device=profile.device,
                 gfx_arch=profile.gfx_arch, torch_device_key=profile.torch_device_key)
    for k, v in overrides.items():
        if k not in Manifest.__dataclass_fields__:
            raise ConfigError(f"unknown manifest field: {k}")
        setattr(m, k, v)
    return m
