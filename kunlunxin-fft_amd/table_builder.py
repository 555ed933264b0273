"""Build the MI355X selector table from live measurements.

MI355X counterpart of the reference's table builder
(scripts/build_selector_table.py; table schema of src/xpu/selector.py:6-41).
For every cell (N, batch, direction) it times the M0 incumbent (fft_dit /
fft_dif and their batch forms) and every legal challenger of the published
design space (config/butterfly_space.json): the radix-4 global-stage flow,
the dense-dot matrix-core flow (the reference's M2 FFT64 on fp32 MFMA), the
single-pass LDS kernel at each elements-per-thread setting (and start
stagger, where it can act), and the four-step at each split, chunking,
schedule (one column group per workgroup, persistent workgroups, or narrow
4-column groups for small batches) and pass-2 row order.  The fastest
challenger is promoted only when it beats the incumbent by at least
GUARD_PCT percent (M0 closure); otherwise the cell keeps M0.  The table is
bound to the device profile hash and the live environment fingerprint, so it
selects only on the stack it was measured on.

The cells are the reference's config-5 sweep, the roofline rows and every
power-of-two batch of every power-of-two N = 16..2^20 up to 2^32 elements.
Above 2^27 elements a cell times the PRUNE_KEEP fastest challengers of the
same N at 2^27 only, and the M0 incumbent 3 times (these cells run last).  A plan the
library refuses at a shape (past one dispatch's 2^32 work-items) is no
candidate, and where the refused plan is M0 the best challenger is promoted.

The same cells, and the roofline rows at twice their batch (where a real
launch moves the C2C row's bytes), are also measured for R2C forward and C2R
inverse with the default norm, against the M0 real flow, and stored as
exact-semantic entries: the real modes of the LDS kernel and the four-step
around a half-length core have their own best settings.

A rebuild never silently regresses a cell the deployed table won: every
cell whose decision changed is re-timed against the previous decision,
alternately, under the current environment, and where the previous one is
faster by more than the guard it is kept as a ``previous_fallbacks`` cell,
bound to this table's environment, profile, precision and device and to the
sha256 of the previous table and of the paired samples
(``carry_previous_fallbacks``); the previous table's own fallback cells are
reconfirmed the same way or dropped with a reason.

Timing: forward C2C complex64 (and the real cells), inputs resident on the GPU.  Cells under
64 MiB: ``reps`` back-to-back executes recorded into one HIP graph, the graph
replayed between HIP events, median of ``rounds`` replays (ms per execute of
device time; a host loop of enqueues would time the host in the launch-bound
cells).  Larger cells: each execute timed alone after an untimed 256 MiB
write elsewhere, median of ``rounds`` x ``reps / 4``.

Usage (on a GPU box):
    python kunlunxin-fft_amd/table_builder.py --out path/selector_table.json [--quick]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

C5_SIZES = [1 << k for k in range(4, 15)]        # the reference's size sweep: N = 16 .. 2^14
C5_BATCHES = [1, 16, 64, 256]
ROOF_SIZES = [1 << k for k in range(10, 21)]      # roofline rows: B = max(64, 2^25/N)
EXTRA_CELLS = [(1 << k, 1) for k in range(15, 21)] + [(1 << 16, 256), (256, 1), (4096, 64)]
# Every power-of-two batch of every power-of-two N from 16 to 2^20, up to
# 2^32 elements (32 GiB of complex64 per buffer): the table answers exact
# (N, batch) keys only, and a shape it does not hold runs the radix-2
# baseline, one launch per stage (at N = 2^20, B = 2, 7x the four-step's time).
DENSE_MAX_LOG_ELEMS = 32
# Above 2^27 elements a cell times only the PRUNE_KEEP fastest challengers of
# the same N (and direction or real semantic) at 2^27 elements, and the M0
# incumbent 3 times after one warm-up (it is several times slower there, far
# outside the 2% guard): every launch streams whole waves of workgroups, so
# the ranking of the 2^27 cell holds, and timing everything at up to 32 GiB
# per buffer would take hours.  These cells are built last.
PRUNE_LOG_ELEMS = 27
PRUNE_KEEP = 3
DENSE_LOG_N = range(4, 21)
# real transforms, default norm: exact-semantic entries at the roofline rows
# (the LDS kernel's real modes and the four-step around a half-length core
# have their own best elements, stagger and split)
REAL_SEMANTICS = (("r2c", "forward"), ("c2r", "inverse"))
REAL_NORM = "backward"
# a runner-up within this many percent of the fastest candidate is timed
# again against it, alternately, this many times each, before a cell is decided
CONFIRM_PCT = 20.0
CONFIRM_ROUNDS = 5


def _sha256_file(path: str) -> str:
    import hashlib

    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def _sha256_json(obj) -> str:
    import hashlib

    return hashlib.sha256(json.dumps(obj, sort_keys=True, separators=(",", ":")).encode()).hexdigest()


def cell_key(entry: dict) -> tuple:
    """(N, batch, direction, transform_type, transform_direction,
    normalization) of an entry; a legacy entry (no semantic triple) is the
    forward C2C cell it was measured on."""
    from kunlunxin_fft_amd.selector import semantic_key_of

    sk = semantic_key_of(entry) or ("c2c", "forward", "backward")
    return (entry["N"], entry["batch"], entry["direction"]) + tuple(sk)


def _geometry(entry: dict) -> tuple:
    """What an entry runs: runner name, block and parameters."""
    return (entry.get("executed"), entry.get("block"), json.dumps(entry.get("params") or {}, sort_keys=True))


def carry_previous_fallbacks(prev: "dict | None", prev_sha: "str | None", table: dict, paired, guard: float,
                             rounds: int = CONFIRM_ROUNDS) -> tuple:
    """Per-cell regression guard of a rebuild (the reference's
    previous-fallback carry and reconfirm, scripts/build_selector_table.py:
    884-1106, under the binding contract of src/xpu/selector.py:260-340).

    ``prev`` is the previously deployed table (its file sha256 ``prev_sha``),
    ``table`` the rebuilt one (its ``entries``, env/profile/precision
    binding and ``env`` device identity already set).  For every rebuilt
    cell whose previous decision (its previous fallback cell, else its exact
    semantic entry, else its legacy entry) runs something else,
    ``paired(rebuilt_entry, previous_entry)`` times the two alternately,
    ``rounds`` times each, under the current environment, and returns
    ``(rebuilt_samples_ms, previous_samples_ms)``.  When the rebuilt choice
    is slower by more than ``guard`` percent (median against median), the
    previous decision is kept as a ``previous_fallbacks`` cell with the exact
    semantic triple and a ``fallback-env-binding-v1`` provenance bound to the
    rebuilt table's environment, profile, precision and device, the previous
    table's sha256 and the sha256 of the paired samples.  The previous
    table's own fallback cells are reconfirmed the same way: kept while they
    still clear the guard, dropped with a reason otherwise.

    Nothing is carried across environments: a previous table bound to
    another env, profile or precision contributes no cell (one reason says
    why), and a previous fallback cell that fails its own binding, or whose
    parameters left the published design space, is dropped with a reason.
    Returns ``(fallbacks, drop_reasons, paired_records)``."""
    from kunlunxin_fft_amd.selector import (DEVICE_IDENTITY_KEYS, FALLBACK_CARRY_CONTRACT,
                                            entry_contract_violations, fallback_binding_violations,
                                            find_entry)

    if not prev:
        return [], [], []
    for key in ("env_hash", "profile_hash", "precision"):
        if not prev.get(key) or prev.get(key) != table.get(key):
            return [], [f"previous table {key} {prev.get(key)!r} != rebuilt table {table.get(key)!r}: "
                        "nothing carried across environments (re-measure instead)"], []
    drops: list[str] = []
    prev_fbs = list(prev.get("previous_fallbacks") or [])
    if prev_fbs and fallback_binding_violations(prev):
        drops += [f"previous fallback cells dropped (binding contract): {m}"
                  for m in fallback_binding_violations(prev)]
        prev = dict(prev, previous_fallbacks=[])
        prev_fbs = []
    ident = {k: (table.get("env") or {}).get(k) for k in DEVICE_IDENTITY_KEYS}
    rebuilt = {cell_key(e): e for e in table.get("entries", [])}
    for fb in prev_fbs:
        if cell_key(fb) not in rebuilt:
            drops.append(f"{cell_key(fb)}: previous fallback cell not in the rebuilt sweep -- dropped")
    fallbacks, records = [], []
    for key, new in rebuilt.items():
        old = find_entry(prev, key[0], key[1], key[2], *key[3:])
        if old is None or _geometry(old) == _geometry(new):
            continue
        was_fallback = any(old is f for f in prev_fbs)
        bad = entry_contract_violations(old)
        if bad:
            if was_fallback:
                drops.append(f"{key}: previous fallback outside the published design space ({bad[0]}) -- dropped")
            continue
        new_s, old_s = paired(new, old)
        new_ms, old_ms = statistics.median(new_s), statistics.median(old_s)
        delta = new_ms / old_ms - 1.0
        rec = {"cell": list(key), "rebuilt": list(_geometry(new)), "previous": list(_geometry(old)),
               "rebuilt_ms": [round(v, 6) for v in new_s], "previous_ms": [round(v, 6) for v in old_s],
               "selector_vs_previous": round(delta, 5)}
        records.append(rec)
        if delta <= guard / 100.0:
            if was_fallback:
                drops.append(f"{key}: rebuilt choice within {delta:+.2%} of the previous fallback "
                             f"(guard {guard}%) -- fallback dropped")
            continue
        fb = json.loads(json.dumps(old))
        fb["transform_type"], fb["transform_direction"], fb["normalization"] = key[3:]
        prov = dict(fb.get("previous_fallback_provenance") or {})
        prov.update({
            "carry_contract": FALLBACK_CARRY_CONTRACT,
            "source_env_hash": table["env_hash"], "source_profile_hash": table["profile_hash"],
            "source_precision": table["precision"], "source_device": ident,
            "source_table_sha256": prev_sha, "source_result_sha256": _sha256_json(rec),
            "paired_confirm": f"table_builder paired re-timing: {rounds} alternating timings each of the rebuilt "
                              "and the previous choice under the rebuilt table's environment",
            "selector_vs_previous": round(delta, 5), "selector_ms": round(new_ms, 6),
            "previous_ms": round(old_ms, 6),
            "regression_reason": f"rebuilt choice {new.get('executed')} slower than the previous deployed "
                                 f"{old.get('executed')} by {delta:+.2%} (> {guard}%)",
        })
        fb["previous_fallback_provenance"] = prov
        fb["reason"] = (f"previous deployed {old.get('executed')} {json.dumps(old.get('params') or {}, sort_keys=True)} "
                        f"kept: the rebuilt choice is {delta:+.1%} slower in paired re-timing")
        fallbacks.append(fb)
    return fallbacks, drops, records


def dense_cells(max_log_elems: int = DENSE_MAX_LOG_ELEMS):
    """(N, batch) for every power-of-two batch up to 2^max_log_elems
    elements, N = 16 .. 2^20."""
    return [(1 << k, 1 << j) for k in DENSE_LOG_N for j in range(0, max_log_elems - k + 1)]


def _unique(cells_):
    seen, out = set(), []
    for c in cells_:
        if c not in seen:
            seen.add(c)
            out.append(c)
    return out


def real_cells(max_log_elems: int = DENSE_MAX_LOG_ELEMS):
    """(N, batch) of the exact-semantic real entries: the roofline rows'
    batch and twice it (the same bytes per launch as the C2C row, which
    bench.py's real rows use), then every dense cell."""
    return _large_last(_unique([(n, b) for n in ROOF_SIZES for b in (max(64, (1 << 25) // n),
                                                                     2 * max(64, (1 << 25) // n))]
                               + dense_cells(max_log_elems)))


def _large_last(cells_):
    """The cells above 2^PRUNE_LOG_ELEMS elements after all the others (their
    challengers come from the 2^PRUNE_LOG_ELEMS cell of the same N)."""
    big = lambda c: c[0] * c[1] > (1 << PRUNE_LOG_ELEMS)
    return [c for c in cells_ if not big(c)] + [c for c in cells_ if big(c)]


def pruned(cands, n: int, b: int, key, top: dict):
    """The challengers to time in cell (n, b): all of them up to
    2^PRUNE_LOG_ELEMS elements; above, those among the PRUNE_KEEP fastest
    that top[key] recorded at 2^PRUNE_LOG_ELEMS (all when none is recorded)."""
    keep = top.get(key)
    if n * b <= (1 << PRUNE_LOG_ELEMS) or not keep:
        return list(cands)
    return [c for c in cands if c[0] in keep]


def guard_gain(inc_ms: float, best) -> float:
    """Percent by which the best challenger beats the M0 incumbent; 100 when
    the library refuses M0 at this shape (inc_ms infinite), -1 with no
    challenger."""
    if best is None or not math.isfinite(best[0]):
        return -1.0
    if not math.isfinite(inc_ms):
        return 100.0
    return (inc_ms - best[0]) / inc_ms * 100.0


def _ms(ms: float):
    """A timing for the sweep record: rounded, or None for a refused plan."""
    return round(ms, 5) if math.isfinite(ms) else None


def _fmt(ms) -> str:
    return "refused" if ms is None else f"{ms:.4f}"


def record_top(timed, n: int, b: int, key, top: dict) -> None:
    """At 2^PRUNE_LOG_ELEMS elements, remember the PRUNE_KEEP fastest labels."""
    ok = [t for t in timed if math.isfinite(t[0])]
    if n * b == (1 << PRUNE_LOG_ELEMS) and ok:
        top[key] = [t[1] for t in sorted(ok, key=lambda t: t[0])[:PRUNE_KEEP]]


def cells(quick: bool = False, max_log_elems: int = DENSE_MAX_LOG_ELEMS):
    out = []
    for n in C5_SIZES:
        for b in C5_BATCHES:
            out.append((n, b))
    for n in ROOF_SIZES:
        out.append((n, max(64, (1 << 25) // n)))
    out += EXTRA_CELLS
    uniq = _large_last(_unique(out + dense_cells(max_log_elems)))
    if quick:
        uniq = [c for c in uniq if c[0] * c[1] <= (1 << 22) or c[1] == 1]
    return uniq


def real_candidates(n: int, b: int, transform_type: str, space):
    """Challengers for a real transform of length n (complex core n/2): the
    LDS kernel's fused real modes (up to a 32768-point core; 32 elements per
    thread only there, where the runner maps 32 to 16 below it), with the
    start stagger in large batches, and the four-step core."""
    sfx = "" if b == 1 else "_batch"
    core = n // 2
    logc = int(math.log2(core)) if core >= 1 else 0
    out = []
    if 1 <= core <= 32768:
        for e in space.lds_elems:
            if e == 32 and logc < 15:
                continue  # real cores below 32768 map 32 to 16
            if logc >= 13 and e < 16:
                continue
            if logc == 15 and e != 32:
                continue
            # below 16 points a thread holds at most the whole core: larger
            # counts than the core repeat the core-sized kernel (16 is the default)
            if e > core and e != 16:
                continue
            stags = [s for s in space.lds_stagger
                     if s == 0 or (e >= 16 and logc >= 9 and n * b >= (1 << 24))]
            for stg in stags:
                params = {"elems": e} if stg == 0 else {"elems": e, "stagger": stg}
                out.append((f"lds_e{e}" + (f"_s{stg}" if stg else ""), "fft_lds_fused" + sfx, 256, params,
                            ("lds-resident", "stockham-radix16", "lds-stockham-single-pass")))
            # the staged form: fewer than 16 threads per transform of the core
            if 1 in space.lds_staged and e != 32 and core // min(e, core) < 16:
                out.append((f"lds_e{e}_st", "fft_lds_fused" + sfx, 256, {"elems": e, "stage": 1},
                            ("lds-resident", "stockham-radix16", "lds-stockham-single-pass")))
    if 256 <= core and core * 2 >= space.fourstep_min_n:
        for n1 in space.fourstep_n1:
            n2 = core // n1
            if n2 < 16 or n2 > 1024 or core % n1:
                continue
            if abs(int(math.log2(n1)) - int(math.log2(n2))) > 2:
                continue
            chunks = [0]
            if b >= 16 and core >= (1 << 14):
                chunks += [c for c in space.fourstep_chunk_rows if c and c < b and core * c * 8 >= (16 << 20)
                           and core * c * 8 <= (256 << 20)]
            for ch in chunks:
                for order in (space.fourstep_pass2_order if b > 1 else (0,)):
                    params = {"n1": n1, "chunk_rows": ch}
                    if order:
                        params["pass2_order"] = order
                    out.append((f"fs_n1_{n1}_c{ch}" + ("_r" if order else ""), "fft_four_step" + sfx, 256,
                                params, ("four-step", "stockham-radix16", "four-step-two-pass")))
                    # the narrow schedule, with the stitch / pre-twiddle as its own launch
                    if 3 in space.fourstep_schedule:
                        out.append((f"fsn_n1_{n1}_c{ch}" + ("_r" if order else ""), "fft_four_step" + sfx, 256,
                                    dict(params, schedule=3),
                                    ("four-step", "stockham-radix16", "four-step-two-pass")))
    return out


def candidates(n: int, b: int, direction: str, space):
    """(label, runner name, block, params, family) for every legal challenger."""
    sfx = "" if b == 1 else "_batch"
    logn = int(math.log2(n))
    out = []
    if n >= 4:
        name = ("fft_dit_radix4" if direction == "dit" else "fft_dif_radix4") + sfx
        out.append((f"m5_{direction}@256", name, 256, {}, ("global-stage", "radix4-scalar", "baseline-global-stage")))
    if n <= space.lds_max_n:
        for e in space.lds_elems:
            if logn >= 13 and e < 16:
                continue
            if logn == 15 and e != 32:
                continue
            if e == 32 and logn < 10:
                continue
            if e > n and e != 16:
                continue
            # the start stagger acts on launches of two or more waves of
            # workgroups with at most four workgroups per CU: 16 or 32
            # elements per thread, in large batches
            stags = [s for s in space.lds_stagger if s == 0 or (e >= 16 and logn >= 10 and n * b >= (1 << 24))]
            for stg in stags:
                params = {"elems": e} if stg == 0 else {"elems": e, "stagger": stg}
                out.append((f"lds_e{e}" + (f"_s{stg}" if stg else ""), "fft_lds_fused" + sfx, 256, params,
                            ("lds-resident", "stockham-radix16", "lds-stockham-single-pass")))
            # the staged form: fewer than 16 threads per transform
            if 1 in space.lds_staged and e != 32 and n // min(e, n) < 16:
                out.append((f"lds_e{e}_st", "fft_lds_fused" + sfx, 256, {"elems": e, "stage": 1},
                            ("lds-resident", "stockham-radix16", "lds-stockham-single-pass")))
    if 2 <= n <= space.dense_max_n:
        # the dense-dot matrix-core flow (the reference's M2 dense-dot FFT64)
        name = ("fft_dit_matrix" if direction == "dit" else "fft_dif_matrix") + sfx
        out.append(("dense_mfma", name, 256, {}, ("matrix-resident", "dense-dot-fft64", "local-fused-tile")))
    if space.fourstep_min_n <= n <= (1 << 20):
        for n1 in space.fourstep_n1:
            n2 = n // n1
            if n2 < 16 or n2 > 1024 or n % n1:
                continue
            # keep splits near square (the other ones are never faster)
            if abs(int(math.log2(n1)) - int(math.log2(n2))) > 2:
                continue
            chunks = [0]
            if b >= 16 and n >= (1 << 14):
                chunks += [c for c in space.fourstep_chunk_rows if c and c < b and n * c * 8 >= (16 << 20)
                           and n * c * 8 <= (256 << 20)]
            l1, l2 = int(math.log2(n1)), int(math.log2(n2))
            for ch in chunks:
                for sched in space.fourstep_schedule:
                    if sched == 2 and not (7 <= l1 <= 9 and 7 <= l2 <= 9 and abs(l1 - l2) <= 1):
                        continue
                    # the reverse pass-2 row order only matters with more than one row
                    for order in (space.fourstep_pass2_order if b > 1 and sched != 2 else (0,)):
                        params = {"n1": n1, "chunk_rows": ch}
                        if sched:
                            params["schedule"] = sched
                        if order:
                            params["pass2_order"] = order
                        out.append((f"{('fs', 'fsp', 'fsf', 'fsn')[sched]}_n1_{n1}_c{ch}" + ("_r" if order else ""),
                                    "fft_four_step" + sfx, 256, params,
                                    ("four-step", "stockham-radix16", "four-step-two-pass")))
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", required=True)
    ap.add_argument("--quick", action="store_true")
    ap.add_argument("--max-log-elems", type=int, default=DENSE_MAX_LOG_ELEMS,
                    help="largest cell of the dense grid, log2 of N x batch (default %(default)s; a smaller "
                         "grid builds faster, and batches past it take its largest batch's decision)")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--rounds", type=int, default=3)
    ap.add_argument("--previous", default=None,
                    help="previously deployed table to guard against (default: the package's "
                         "config/selector_table.json when present)")
    ap.add_argument("--no-carry", action="store_true", help="write no previous_fallbacks cells")
    args = ap.parse_args()

    import torch

    sys.path.insert(0, ROOT)
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    from kunlunxin_fft_amd import envcheck
    from kunlunxin_fft_amd.config import DesignSpace, DeviceProfile
    from kunlunxin_fft_amd.entry import ExecutionPlan
    from kunlunxin_fft_amd.runner import get_native_plan, output_spec, time_native_graph, workspace_for
    from kunlunxin_fft_amd.selector import GUARD_PCT, TABLE_PATH

    space = DesignSpace.load()
    env = envcheck.collect()
    env_hash = envcheck.current_env_hash()
    if env is None or env_hash is None:
        print("environment fingerprint unknown: refusing to build a table", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)

    # Cells of 64 MiB and more: each timed execute follows an untimed write of
    # 256 MiB elsewhere, as one size follows another in an application (and
    # in bench.py's step).  Back-to-back repeats would rewrite an output that
    # stays in the 256 MB MALL and absorbs the writes, which favours
    # configurations for a reason no real workload has.  Smaller cells are
    # timed back to back: they live in the MALL in any use.
    flush = torch.empty(1 << 26, dtype=torch.float32, device=dev)  # 256 MiB

    def time_runner(name, n, b, block, params, x, tt="c2c", td="forward", few=False):
        try:
            np_ = get_native_plan(name, n, b, tt, td, "backward", block, params, 0)
        except ValueError as exc:
            # a plan the library refuses for this shape (a launch past one
            # dispatch's 2^32 work-items): not a candidate here
            print(f"  {name} {params} refused at N={n} B={b} {tt}: {exc}", flush=True)
            return math.inf
        shape, dt = output_spec(tt, n, b)
        out = torch.empty(shape, dtype=dt, device=dev)
        ws = workspace_for(np_, dev)
        wp = ws.data_ptr() if ws is not None else 0

        def execute():
            np_.execute_ws(x.data_ptr(), out.data_ptr(), wp, np_.ws_bytes, stream.cuda_stream)

        for _ in range(1 if few else 3):
            execute()
        res = []
        if n * b * (8 if tt == "c2c" else 4) >= (64 << 20):
            # few: the M0 incumbent of a pruned cell, 3 timings
            for _ in range(1 if few else args.rounds):
                for _ in range(3 if few else max(3, args.reps // 4)):
                    flush.fill_(1.0)
                    s = torch.cuda.Event(enable_timing=True)
                    e = torch.cuda.Event(enable_timing=True)
                    s.record(stream)
                    execute()
                    e.record(stream)
                    e.synchronize()
                    res.append(s.elapsed_time(e))
            return statistics.median(res)
        # below 64 MiB: device time of back-to-back executes replayed from a
        # HIP graph (a host loop would time the host's enqueue rate in the
        # launch-bound cells)
        return time_native_graph(np_, x, out, ws, reps=args.reps, rounds=args.rounds)

    def confirm(timed, n, b, x, row, tt="c2c", td="forward"):
        """The fastest candidate, confirmed: when the runner-up is within
        CONFIRM_PCT of it, both are timed again, alternately, CONFIRM_ROUNDS
        times each, and the lower median of those re-timings decides (one
        noisy median in a launch-bound cell must not pick a kernel that is
        slower on average).  The re-timings are recorded in the sweep row."""
        timed = sorted((t for t in timed if math.isfinite(t[0])), key=lambda t: t[0])
        if not timed:
            return None
        if len(timed) < 2 or timed[1][0] > timed[0][0] * (1 + CONFIRM_PCT / 100.0):
            return timed[0]
        again = {0: [], 1: []}
        for _ in range(CONFIRM_ROUNDS):
            for i in (0, 1):
                ms_, _, name_, block_, params_, _ = timed[i]
                again[i].append(time_runner(name_, n, b, block_, params_, x, tt, td))
        med = {i: statistics.median(v) for i, v in again.items()}
        row["confirm"] = {timed[i][1]: round(med[i], 5) for i in (0, 1)}
        w = 0 if med[0] <= med[1] else 1
        return (med[w],) + tuple(timed[w][1:])

    entries, sweep = [], []
    top = {}  # (n, direction or transform type) -> fastest labels at 2^PRUNE_LOG_ELEMS
    t_start = time.time()
    for (n, b) in cells(args.quick, args.max_log_elems):
        shape = (n,) if b == 1 else (b, n)
        x = torch.randn(shape, dtype=torch.complex64, device=dev, generator=gen)
        for direction in ("dit", "dif"):
            inc_name = ("fft_dit" if direction == "dit" else "fft_dif") + ("" if b == 1 else "_batch")
            inc_ms = (time_runner(inc_name, n, b, 256, {}, x, few=n * b > (1 << PRUNE_LOG_ELEMS))
                      if n >= 2 else float("inf"))
            row = {"N": n, "batch": b, "direction": direction, f"m0_{direction}@256": _ms(inc_ms)}
            timed = []
            for label, name, block, params, fam in pruned(candidates(n, b, direction, space), n, b,
                                                          (n, direction), top):
                ms = time_runner(name, n, b, block, params, x)
                row[label] = _ms(ms)
                timed.append((ms, label, name, block, params, fam))
            record_top(timed, n, b, (n, direction), top)
            best = confirm(timed, n, b, x, row)
            sweep.append(row)
            gain = guard_gain(inc_ms, best)
            inc_ms = inc_ms if math.isfinite(inc_ms) else None
            if best is not None and gain >= GUARD_PCT:
                ms, label, name, block, params, (real, unit, flow_id) = best
                entry = {"N": n, "batch": b, "direction": direction, "incumbent_ms": inc_ms,
                         "incumbent_block": 256, "challenger_ms": ms,
                         "evidence": {"incumbent": f"m0_{direction}@256", "challenger": label,
                                      "gain_pct": round(gain, 2)},
                         "reason": f"challenger {label} beats M0 incumbent m0_{direction}@256 by "
                                   f"{gain:.1f}% (>= {GUARD_PCT}%)",
                         "block": block, "flow_id": flow_id, "flow_realization": real,
                         "processing_unit": unit, "params": dict(params), "executed": name}
            else:
                entry = {"N": n, "batch": b, "direction": direction, "incumbent_ms": inc_ms,
                         "incumbent_block": 256, "challenger_ms": best[0] if best else None,
                         "evidence": {"incumbent": f"m0_{direction}@256",
                                      "challenger": best[1] if best else None,
                                      "gain_pct": round(gain, 2)},
                         "reason": f"no challenger beats M0 by {GUARD_PCT}%; M0 kept",
                         "block": 256, "flow_id": "baseline-global-stage",
                         "flow_realization": "global-stage", "processing_unit": "radix2-scalar",
                         "params": {}, "executed": inc_name}
            if b > 1:
                entry["params"]["variant"] = "folded"
            entries.append(entry)
            print(f"N={n:>8} B={b:>6} {direction}: M0 {_fmt(inc_ms)} ms, best {best[1] if best else '-'} "
                  f"{best[0] if best else float('nan'):.4f} ms ({gain:+.1f}%) -> {entry['executed']} "
                  f"[{time.time() - t_start:.0f}s]", flush=True)
        del x
    # ---- real transforms at the roofline rows: exact-semantic entries
    for n, b in ([] if args.quick else real_cells(args.max_log_elems)):
        for tt, td in REAL_SEMANTICS:
            if tt == "r2c":
                x = torch.randn((b, n), dtype=torch.float32, device=dev, generator=gen)
            else:
                x = torch.randn((b, n // 2 + 1), dtype=torch.complex64, device=dev, generator=gen)
            inc_name = "fft_dit" if b == 1 else "fft_dit_batch"
            inc_ms = time_runner(inc_name, n, b, 256, {}, x, tt, td, few=n * b > (1 << PRUNE_LOG_ELEMS))
            row = {"N": n, "batch": b, "direction": "dit", "transform_type": tt, "m0_dit@256": _ms(inc_ms)}
            timed = []
            for label, name, block, params, fam in pruned(real_candidates(n, b, tt, space), n, b, (n, tt), top):
                ms = time_runner(name, n, b, block, params, x, tt, td)
                row[label] = _ms(ms)
                timed.append((ms, label, name, block, params, fam))
            record_top(timed, n, b, (n, tt), top)
            best = confirm(timed, n, b, x, row, tt, td)
            sweep.append(row)
            gain = guard_gain(inc_ms, best)
            inc_ms = inc_ms if math.isfinite(inc_ms) else None
            sem = {"transform_type": tt, "transform_direction": td, "normalization": REAL_NORM}
            if best is not None and gain >= GUARD_PCT:
                ms, label, name, block, params, (real, unit, flow_id) = best
                entry = {"N": n, "batch": b, "direction": "dit", **sem, "incumbent_ms": inc_ms,
                         "incumbent_block": 256, "challenger_ms": ms,
                         "evidence": {"incumbent": "m0_dit@256", "challenger": label, "gain_pct": round(gain, 2)},
                         "reason": f"{tt}: challenger {label} beats M0 incumbent m0_dit@256 by "
                                   f"{gain:.1f}% (>= {GUARD_PCT}%)",
                         "block": block, "flow_id": flow_id, "flow_realization": real,
                         "processing_unit": unit, "params": dict(params), "executed": name}
                if b > 1:
                    entry["params"]["variant"] = "folded"
                entries.append(entry)
            print(f"{tt} N={n:>8} B={b:>6}: M0 {_fmt(inc_ms)} ms, best {best[1] if best else '-'} "
                  f"{best[0] if best else float('nan'):.4f} ms ({gain:+.1f}%) [{time.time() - t_start:.0f}s]",
                  flush=True)
            del x

    table = {
        "schema_version": 1, "device": DeviceProfile.load().device,
        "profile_hash": DeviceProfile.load().hash(), "env_hash": env_hash,
        "env": {**env, "device_model": env["gfx_arch"]},
        "precision": "fp32", "guard_pct": GUARD_PCT,
        "selection_semantics": "median of rounds x (reps back-to-back executes replayed from a HIP graph / reps), "
                               "HIP events; "
                               "cells of 64 MiB and more: each execute after an untimed 256 MiB write; "
                               "forward C2C complex64 (legacy entries, answering every semantic), plus "
                               "exact-semantic R2C / C2R entries (norm backward); cells: the reference's "
                               "config-5 sweep, the roofline rows and every power-of-two batch of every "
                               "power-of-two N = 16 .. 2^20 up to 2^32 elements (above 2^27: the 3 fastest "
                               "challengers of the same N at 2^27, and M0 timed 3 times)",
        "sources": ["kunlunxin-fft_amd/table_builder.py live sweep"],
        "entries": entries, "previous_fallbacks": [],
    }

    # ---- per-cell regression guard against the previously deployed table
    prev_path = args.previous or TABLE_PATH
    prev = prev_sha = None
    if not args.no_carry and os.path.exists(prev_path):
        try:
            prev = pkg.load_table(prev_path)
            prev_sha = _sha256_file(prev_path)
        except pkg.ConfigError as e:
            print(f"previous table {prev_path} refused by the loader ({e}); nothing carried", file=sys.stderr)
            prev = None
    if prev is not None:
        def paired(new_e, old_e):
            n, b, d = new_e["N"], new_e["batch"], new_e["direction"]
            tt, td, _ = cell_key(new_e)[3:]
            if tt == "r2c":
                x = torch.randn((b, n), dtype=torch.float32, device=dev, generator=gen)
            else:
                m = n // 2 + 1 if tt == "c2r" else n
                x = torch.randn((m,) if b == 1 else (b, m), dtype=torch.complex64, device=dev, generator=gen)
            got = ([], [])
            for _ in range(CONFIRM_ROUNDS):
                for i, e in enumerate((new_e, old_e)):
                    got[i].append(time_runner(e["executed"], n, b, e["block"], e.get("params") or {}, x, tt, td))
            return got

        fbs, drops, records = carry_previous_fallbacks(prev, prev_sha, table, paired, GUARD_PCT)
        table["previous_table_sha256"] = prev_sha
        table["previous_fallbacks"] = fbs
        if drops:
            table["previous_fallbacks_dropped"] = drops
        sweep.append({"paired_with_previous": records})
        for fb in fbs:
            print(f"previous fallback kept: {cell_key(fb)} -> {fb['executed']} "
                  f"({fb['previous_fallback_provenance']['selector_vs_previous']:+.2%})", flush=True)
        for m in drops:
            print(f"previous_fallbacks: {m}", file=sys.stderr, flush=True)
    with open(args.out, "w") as f:
        json.dump(table, f, indent=1)
    with open(os.path.splitext(args.out)[0] + "_sweep.json", "w") as f:
        json.dump(sweep, f, indent=1)
    # the table must pass its own loader's contract
    pkg.load_table(args.out)
    print(f"wrote {args.out} ({len(entries)} entries)", flush=True)
    del ExecutionPlan
    return 0


if __name__ == "__main__":
    sys.exit(main())
