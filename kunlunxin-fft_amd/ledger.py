"""Phase and launch ledger (reference src/xpu/ledger.py, same names and
contract).  Three kinds of evidence, each labelled and never mixed:

* fresh measured -- ``PhaseLedger`` times the phases of ``execute_fft_plan``
  (reference ledger.py:64-124) with a device synchronize around each phase.
  That is attribution only: headline timings run with no ledger active,
  where ``phase`` returns one shared no-op context and the plan-reuse fast
  path of ``execute_fft_plan`` stays on.
* analytic estimate -- ``launch_ledger`` (reference ledger.py:163-262) gives
  the launches, HBM bytes and flops of a plan from the rules the native
  library applies when it creates the plan (flow resolution, four-step
  split and chunking, which real-transform epilogues run fused).  They are
  not hardware counters; the HBM bytes that kernels really move come from
  rocprofv3's FETCH_SIZE / WRITE_SIZE.
* summary-derived -- ``batch_fill_analysis`` (reference ledger.py:302-346)
  re-reads per-cell medians to show per-point cost against batch.

Here every real-transform epilogue, the inverse direction and the
normalisation run inside the core's kernels (their loads and stores), so
``execute_fft_plan`` has two phases, ``plan-validate`` and ``core-invoke``,
where the reference's real-compat path has up to six.
"""
from __future__ import annotations

import statistics
import time
from contextvars import ContextVar

from . import flows, native

KIND_FRESH = "fresh measured (phase timers; extra synchronize added)"
KIND_ANALYTIC = "analytic estimate (native plan rules; not hardware counters)"
KIND_SUMMARY = "summary-derived (per-cell medians)"

ACTIVE: ContextVar = ContextVar("mfft_phase_ledger", default=None)

# Runner name -> the reference's lowering family for that name
# (reference ledger.py:34-49); kept beside this library's own flow so that
# reports of either library line up.  The counts below are this library's.
REFERENCE_FAMILIES = {
    "fft_dit": "baseline_m0_rank1_loop",
    "fft_dif": "baseline_m0_rank1_loop",
    "fft_dit_batch": "incumbent_m4_folded",
    "fft_dif_batch": "incumbent_m4_folded",
    "fft_dit_radix4": "m5_batch",
    "fft_dif_radix4": "m5_batch",
    "fft_dit_radix4_batch": "m5_batch",
    "fft_dif_radix4_batch": "m5_batch",
    "fft_dit_matrix": "m2_batch",
    "fft_dif_matrix": "m2_batch",
    "fft_dit_matrix_batch": "m2_batch",
    "fft_dif_matrix_batch": "m2_batch",
    "fft_dit_matrix_packet_batch": "m2_packet",
    "fft_dif_matrix_packet_batch": "m2_packet",
}

# native flow -> (family, efficiency class)
_FLOW_FAMILY = {
    native.FLOW_RADIX2_DIT: ("stage-radix2", "hbm round trip per radix-2 stage"),
    native.FLOW_RADIX2_DIF: ("stage-radix2", "hbm round trip per radix-2 stage"),
    native.FLOW_RADIX4_DIT: ("stage-radix4", "hbm round trip per radix-4 stage"),
    native.FLOW_RADIX4_DIF: ("stage-radix4", "hbm round trip per radix-4 stage"),
    native.FLOW_LDS_FUSED: ("lds-single-pass", "one hbm read and write; stages in LDS"),
    native.FLOW_FOUR_STEP: ("four-step-two-pass", "two hbm round trips; each pass in LDS"),
    native.FLOW_DENSE_MFMA: ("dense-mfma", "one hbm read and write; fp32 matrix-core dot"),
}

MAX_LDS_CORE = 1 << 15  # the single-pass kernel's longest core


def _sync() -> None:
    import torch

    torch.cuda.synchronize()


class PhaseLedger:
    """Per-phase wall times of one context (reference ledger.py:64-124).

    ``sync=True`` synchronizes the device before and after every phase:
    right for attribution, wrong for headline timing.
    """

    def __init__(self, sync: bool = True):
        self.sync = sync
        self.phases: list[dict] = []

    def phase(self, name: str):
        return _Phase(self, name)

    def summary(self) -> dict:
        """Calls, mean, median and max per phase, in first-seen order, and
        the phases that raised."""
        by: dict[str, list[float]] = {}
        errors = []
        for p in self.phases:
            by.setdefault(p["name"], []).append(p["ms"])
            if p["error"]:
                errors.append({"name": p["name"], "error": p["error"]})
        return {
            "kind": KIND_FRESH,
            "sync_added": self.sync,
            "phases": {k: {"calls": len(v), "mean_ms": statistics.fmean(v), "p50_ms": statistics.median(v),
                           "max_ms": max(v)} for k, v in by.items()},
            "phase_order": list(by),
            "errors": errors,
            "note": "attribution mode: every phase is bracketed by a device synchronize; not comparable "
                    "with headline timings, which run with no ledger active",
        }


class _Phase:
    """One timed phase; a phase that raises is recorded with its error and
    the exception goes on."""

    __slots__ = ("led", "name", "t0")

    def __init__(self, led: PhaseLedger, name: str):
        self.led, self.name = led, name

    def __enter__(self):
        if self.led.sync:
            _sync()
        self.t0 = time.perf_counter()
        return None

    def __exit__(self, et, ev, tb):
        if self.led.sync:
            try:
                _sync()
            except Exception:  # noqa: BLE001 - keep the record of the failing phase
                pass
        self.led.phases.append({"name": self.name, "ms": (time.perf_counter() - self.t0) * 1e3,
                                "error": None if et is None else f"{et.__name__}: {ev}"})
        return False


class _Noop:
    """The shared context of every phase while no ledger is active."""

    __slots__ = ()

    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NOOP = _Noop()


def phase(name: str):
    """Record ``name`` on the active ledger; the shared no-op otherwise."""
    led = ACTIVE.get()
    if led is None:
        return _NOOP
    return led.phase(name)


def current_ledger() -> PhaseLedger | None:
    return ACTIVE.get()


def _row_bytes(transform_type: str, n: int) -> tuple[int, int]:
    """HBM bytes of one input row and one output row."""
    if transform_type == "r2c":
        return 4 * n, 8 * (n // 2 + 1)
    if transform_type == "c2r":
        return 8 * (n // 2 + 1), 4 * n
    return 8 * n, 8 * n


def _resolve(executed: str, n: int, batch: int, transform_type: str, block, params: dict) -> dict:
    """The flow and geometry the native library builds for a plan, by the
    rules of mfft_plan_create_ex: FLOW_AUTO is the LDS kernel up to a core
    of 2^15 and the four-step above; the four-step splits the core as
    n1 = 2^floor(log2(core)/2) unless n1 is given, launches 2 passes per
    chunk of rows, and fuses the real stitch / pre-twiddle into its passes
    in schedule 0; every other flow runs a real transform's stitch or
    pre-twiddle as one extra launch (one per chunk of a chunked four-step)."""
    flow, prm = flows.flow_params(executed, n, transform_type, block, params)
    core = n // 2 if transform_type in ("r2c", "c2r") else n
    logc = core.bit_length() - 1
    if flow == native.FLOW_AUTO:
        flow, prm = (native.FLOW_LDS_FUSED, ()) if core <= MAX_LDS_CORE else (native.FLOW_FOUR_STEP, ())
    real = transform_type != "c2c"
    g = {"flow": flow, "core": core, "logc": logc, "real": real}
    if flow in (native.FLOW_RADIX2_DIT, native.FLOW_RADIX2_DIF):
        core_launches, passes = logc, logc
    elif flow in (native.FLOW_RADIX4_DIT, native.FLOW_RADIX4_DIF):
        core_launches = passes = logc // 2 + (logc & 1)
    elif flow == native.FLOW_FOUR_STEP:
        prm = tuple(prm) + (0,) * (4 - len(prm))
        n1 = int(prm[0]) or 1 << (logc // 2)
        chunk = int(prm[1]) if 0 < int(prm[1]) < batch else batch
        sched = int(prm[2])
        nc = -(-batch // chunk)
        core_launches, passes = 2 * nc, 2
        g.update(n1=n1, n2=core // n1, chunk_rows=chunk, chunks=nc, schedule=sched)
    else:  # LDS, dense
        core_launches, passes = 1, 1
    fused_real = real and (flow == native.FLOW_LDS_FUSED
                           or (flow == native.FLOW_FOUR_STEP and g["schedule"] == 0))
    if not real or fused_real:
        real_launches = 0
    elif flow == native.FLOW_FOUR_STEP and g["schedule"] != 2:
        real_launches = g["chunks"]
    else:
        real_launches = 1
    g.update(core_launches=core_launches, real_launches=real_launches, passes=passes, fused_real=fused_real)
    return g


def _real_ops(transform_type: str, n: int, batch: int, fused: bool, inverse: bool, scaled: bool) -> list[dict]:
    """The reference's real-compat / inverse / scale ops (reference
    ledger.py:192-261), as this library runs them: fused ops move no bytes
    of their own; an unfused stitch or pre-twiddle is one kernel over the
    half spectrum."""
    half, zrow = 8 * (n // 2 + 1) * batch, 8 * (n // 2) * batch
    ops = []
    if transform_type == "r2c":
        ops.append({"op": "real-input pack (none: the core loads x as n/2 complex pairs)",
                    "fused": True, "in_bytes": 0, "out_bytes": 0})
        ops.append({"op": "half-spectrum stitch (bin k with bin n/2-k, scale in the store)",
                    "fused": fused, "in_bytes": 0 if fused else zrow, "out_bytes": 0 if fused else half})
    elif transform_type == "c2r":
        ops.append({"op": "half-spectrum pre-twiddle (bin k with bin n/2-k)",
                    "fused": fused, "in_bytes": 0 if fused else half, "out_bytes": 0 if fused else zrow})
        ops.append({"op": "real-output interleave (none: the core stores n/2 complex as n reals)",
                    "fused": True, "in_bytes": 0, "out_bytes": 0})
    elif inverse:
        ops.append({"op": "inverse direction (twiddle sign; no conjugate pass)",
                    "fused": True, "in_bytes": 0, "out_bytes": 0})
    if scaled:
        ops.append({"op": "normalization scale (in the final store)", "fused": True, "in_bytes": 0, "out_bytes": 0})
    for o in ops:
        o["kind"] = "analytic estimate"
    return ops


def launch_ledger(plan) -> dict:
    """Analytic launches / HBM bytes / flops of one resolved plan
    (reference ledger.py:163-262).

    ``gm_bytes`` counts the input and output streams and every round trip
    of an intermediate through HBM (four-step Z, stage-flow passes, unfused
    epilogues); twiddle and matrix tables, which sit in the caches, are not
    counted.  ``flops`` is the usual 5 N log2 N per complex core transform
    (the real transforms: that of their N/2 core plus 10 per bin pair of the
    stitch).  A composition around the vendor core runs rocFFT's launches,
    which stay opaque: ``available`` False, never invented.
    """
    executed = getattr(plan, "executed", None)
    n, batch = int(plan.n), int(plan.batch)
    params = dict(getattr(plan, "params", None) or {})
    ttype = getattr(plan, "transform_type", "c2c")
    tdir = getattr(plan, "transform_direction", "forward")
    norm = getattr(plan, "norm", "backward")
    out = {"kind": KIND_ANALYTIC, "executed": executed, "estimate": True,
           "reference_family": REFERENCE_FAMILIES.get(executed)}
    if executed == "run_hybrid" and params.get("core") == "vendor":
        out.update(family=None, available=False, real_compat_ops=[],
                   why="composition around the vendor core: rocFFT's sub-transform launches are opaque here; "
                       "the sub-transform shapes and counts are in the HybridPlan's plan_ledger")
        return out
    if executed not in flows.RUNNER_FLOWS:
        out.update(family=None, available=False, real_compat_ops=[],
                   why=f"no registered lowering family for {executed!r}")
        return out
    g = _resolve(executed, n, batch, ttype, getattr(plan, "block", None), params)
    family, eff = _FLOW_FAMILY[g["flow"]]
    if g["flow"] == native.FLOW_FOUR_STEP and g["schedule"] == 2:
        family, eff = "four-step-fused-l2", "one hbm read and write when the L2 ring holds Z"
    core, zrow = g["core"], 8 * g["core"] * batch
    in_row, out_row = _row_bytes(ttype, n)
    alg = (in_row + out_row) * batch
    if g["fused_real"] or not g["real"]:
        core_io = alg
    else:
        core_io = 2 * zrow
    if g["flow"] in (native.FLOW_RADIX2_DIT, native.FLOW_RADIX2_DIF, native.FLOW_RADIX4_DIT,
                     native.FLOW_RADIX4_DIF):
        gm = g["passes"] * 2 * zrow  # every stage reads and writes the core rows
    elif g["flow"] == native.FLOW_FOUR_STEP and g["schedule"] != 2:
        gm = core_io + 2 * zrow
    else:
        gm = core_io
    from .entry import norm_scale

    ops = _real_ops(ttype, n, batch, g["fused_real"], tdir == "inverse", norm_scale(n, tdir, norm) != 1.0)
    gm += sum(o["in_bytes"] + o["out_bytes"] for o in ops)
    logc = g["logc"]
    flops = 5.0 * core * logc * batch + (10.0 * (core // 2 + 1) * batch if g["real"] else 0.0)
    out.update(family=family, available=True, flow=native.FLOW_NAMES[g["flow"]],
               launches=g["core_launches"] + g["real_launches"], core_launches=g["core_launches"],
               epilogue_launches=g["real_launches"], gm_bytes=int(gm), algorithmic_bytes=int(alg),
               traffic_over_algorithmic=round(gm / alg, 4), flops=flops, efficiency=eff,
               real_compat_ops=ops)
    for k in ("n1", "n2", "chunk_rows", "schedule"):
        if k in g:
            out[k] = g[k]
    return out


def measure_phases(plan, x, trials: int = 30, warmup: int = 5) -> dict:
    """Fresh-measured phase breakdown of ``execute_fft_plan`` on the device
    (reference ledger.py:265-299): ``warmup`` untimed calls, then ``trials``
    calls each between two synchronizes, with the ledger active."""
    import torch

    from .entry import execute_fft_plan

    led = PhaseLedger(sync=True)
    tok = ACTIVE.set(led)
    walls = []
    try:
        for _ in range(max(1, warmup)):
            execute_fft_plan(plan, x)
            torch.cuda.synchronize()
        led.phases.clear()
        for _ in range(max(1, trials)):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            execute_fft_plan(plan, x)
            torch.cuda.synchronize()
            walls.append((time.perf_counter() - t0) * 1e3)
    finally:
        ACTIVE.reset(tok)
    out = led.summary()
    out["trials"] = len(walls)
    out["trial_wall_p50_ms"] = statistics.median(walls)
    out["trial_wall_mean_ms"] = statistics.fmean(walls)
    out["phase_sum_mean_ms"] = sum(v["mean_ms"] for v in out["phases"].values())
    out["inter_phase_host_overhead_ms"] = out["trial_wall_mean_ms"] - out["phase_sum_mean_ms"]
    return out


def batch_fill_analysis(cases: list[dict], n_values: list[int] | None = None) -> list[dict]:
    """Per-point cost against batch for each (N, semantic) with at least
    three batch points (reference ledger.py:302-346).  ``cases`` hold
    ``N``, ``batch``, ``semantic``, ``selector_ms`` and ``vendor_ms``; a
    case missing either time is skipped.  ``poor_batch_fill`` is set when
    the selector's per-point cost at the largest batch exceeds 1.5x that at
    the smallest."""
    groups: dict = {}
    for c in cases:
        if c.get("selector_ms") is None or c.get("vendor_ms") is None:
            continue
        if n_values and c["N"] not in n_values:
            continue
        groups.setdefault((c["N"], c["semantic"]), {})[c["batch"]] = c
    out = []
    for (n, semantic), by_b in sorted(groups.items()):
        if len(by_b) < 3:
            continue
        pts = [{"B": b, "selector_ms": by_b[b]["selector_ms"], "vendor_ms": by_b[b]["vendor_ms"],
                "selector_us_per_point": by_b[b]["selector_ms"] * 1e3 / (n * b),
                "vendor_us_per_point": by_b[b]["vendor_ms"] * 1e3 / (n * b)} for b in sorted(by_b)]
        s0, v0 = pts[0]["selector_us_per_point"], pts[0]["vendor_us_per_point"]
        growth = pts[-1]["selector_us_per_point"] / s0 if s0 else None
        vgrowth = pts[-1]["vendor_us_per_point"] / v0 if v0 else None
        out.append({
            "N": n, "semantic": semantic, "kind": KIND_SUMMARY, "points": pts,
            "selector_per_point_growth_smallest_to_largest_B": growth,
            "vendor_per_point_growth_smallest_to_largest_B": vgrowth,
            "poor_batch_fill": bool(growth is not None and growth > 1.5),
            "conclusion_scope": "per-point wall time from per-cell medians; a fill proxy only -- no worker/wave "
                                "hardware counters are read here (rocprofv3 holds those)",
        })
    return out
