"""Benchmark: C2C complex64 GB/s and % of HBM peak, N = 2^10..2^20, plus the
p50 latency at N=2048 B=1 (the reference's headline metric), on one MI355X.

One step = one forward C2C complex64 transform (through the public plan API:
``plan_fft`` with the device profile -> ``execute_fft_plan``) of every size
N = 2^10 .. 2^20 at B = max(64, 2^25 / N) rows -- 256 MiB in and 256 MiB out
per size (512 MiB each way at 2^20, where B = 64), no less than the 256 MB
Infinity Cache.  Inputs are synthetic
(iid N(0,1) real/imag parts from a fixed device-side seed) and resident in
HBM before the timed region.  ``value`` = algorithmic bytes of all K steps
(16*N*B per transform) / timed wall time, in GB/s.

Output: the last stdout line is one compact JSON record (``compact_line``,
a few KB: the contract keys, ``roofline``, ``cpu_baseline``, the latency
p50s, per-size ``[N, GB/s, frac]`` rows, configs 2-4 rows, a config-5
summary and the provenance hashes); progress and per-cell lines go to
stderr before it, and the full record below (per-launch times, vendor
columns, every config-5 cell) to ``--detail-out``
(``gpurun_out/bench_detail.json`` by default).

Also reported:
* ``provenance``: device profile and live environment hashes, the sha256
  of the selector/composition tables and their own bindings, of the kernel
  sources and of the built library, and the commit when one is present;
* ``roofline``: the dominant flow (the size whose launches take the largest
  share of a step): the transforms' algorithmic bytes (16 N per row) over the
  sum of the durations of all launches of one execute (both four-step passes
  of every chunk together; HIP events on the stream the kernels run on),
  against 8 TB/s; ``traffic`` = the HBM bytes of the same launches from the
  committed rocprofv3 PMC summary (profiles/pmc_traffic.json) when present,
  else null, and its ratio to the algorithmic bytes;
* ``per_size``: GB/s, fraction of peak and GFLOP/s (5 N log2 N per transform)
  per N: the median of 100 executes of each size (HIP events, in the step's
  cyclic order, after the timed steps as warm-up), and each launch's median
  duration over 20 timed executes;
* ``latency_n2048_b1``: the reference protocol (warmup 5, 5 x 32 trials,
  device sync per trial, pooled p50 and MAD, scripts/issue10_wp3_holdout.py:176-190)
  for execute_fft_plan, plus the kernel-only event p50 and the per-transform
  time of 64 executes recorded into one HIP graph and replayed;
* ``config2``: latency and GB/s of the reference's small-batch configuration (N in {1024, 2048}, B in
  {16, 64}); ``config3``: the same for inverse C2C, R2C and C2R at N in {256, 4096}, B in {1, 64}
  (real transforms count 4N + 8(N/2+1) bytes per row); ``config4``: the same for N=2^20 B=1 and
  N=2^16 B=256;
* ``real_per_size``: R2C forward and C2R inverse at the same N and twice the
  batch, i.e. the same bytes per launch as the C2C row (the selected plans),
  GB/s and fraction of peak from HIP events in cyclic order, counting
  4N + 8(N/2+1) bytes per row;
* ``per_size[].vendor_*``: torch.fft.fft (rocFFT) on the same inputs, a
  comparison column only;
* ``config5``: the selector sweep (N = 16 .. 2^14, B in {1, 16, 64, 256}):
  per cell the device time per execute (executes replayed back to back from
  a HIP graph) of the selected plan, the M0 incumbent and the dense-dot MFMA
  candidate (the reference's M2 flow), and whether the selected plan clears
  the 2% promotion guard in this run;
* ``cpu_baseline``: the reference's own CPU FFT (butterfly::fft_dit built
  into oracle/_ref; the C restatement when that build is absent) on one core,
  on a bounded sample -- 16 transforms of each N = 2^10..2^20 -- median of 5,
  plus the same rows spread over up to 16 host threads (``all_cores``).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import gc
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_GBPS = 8000.0
SIZES = [1 << k for k in range(10, 21)]
METRIC = "C2C complex64 GB/s & % HBM peak, N=2^10-2^20; p50 latency N=2048 B=1"
WORKLOAD = ("forward C2C complex64 via plan_fft/execute_fft_plan, N=2^10..2^20, B=max(64, 2^25/N) "
            "per N (256 MiB in + 256 MiB out per N, 512 MiB each way at 2^20); one step = all 11 sizes")
DEFAULT_DETAIL = os.path.join(ROOT, "gpurun_out", "bench_detail.json")
# The stdout line is read from the tail of the process output; everything
# else goes to stderr and to the detail file.
LINE_LIMIT = 4096


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _sha16_files(paths) -> "str | None":
    import hashlib

    h = hashlib.sha256()
    seen = False
    for p in paths:
        try:
            with open(p, "rb") as f:
                h.update(os.path.basename(p).encode() + b"\0" + f.read())
            seen = True
        except OSError:
            continue
    return h.hexdigest()[:16] if seen else None


def provenance(pkg, profile_hash: str) -> dict:
    """What a row is tied to: the device profile and live environment hashes,
    the selector and composition tables the plans came from (file sha256 and
    the table's own bindings), the kernel sources and the built library, and
    the commit when a git checkout is present, else the one the library's
    build recorded."""
    import glob
    import subprocess

    from kunlunxin_fft_amd import envcheck
    from kunlunxin_fft_amd.config import CONFIG_DIR

    pdir = os.path.dirname(pkg.__file__)
    sel = os.path.join(CONFIG_DIR, "selector_table.json")
    try:
        with open(sel) as f:
            tab = json.load(f)
    except (OSError, ValueError):
        tab = {}
    commit = None
    try:
        r = subprocess.run(["git", "rev-parse", "--short=12", "HEAD"], cwd=ROOT, capture_output=True,
                           text=True, timeout=10)
        commit = r.stdout.strip() or None if r.returncode == 0 else None
    except (OSError, subprocess.SubprocessError):
        commit = None
    try:
        with open(os.path.join(pdir, "libmfft.build.json")) as f:
            built = json.load(f)
    except (OSError, ValueError):
        built = {}
    csrc = _sha16_files(sorted(glob.glob(os.path.join(pdir, "csrc", "*"))))
    return {"profile_hash": profile_hash, "env_hash": envcheck.current_env_hash(),
            "table_sha16": _sha16_files([sel]),
            "table_profile_hash": tab.get("profile_hash"), "table_env_hash": tab.get("env_hash"),
            "composition_sha16": _sha16_files([os.path.join(CONFIG_DIR, "composition_table.json")]),
            "csrc_sha16": csrc,
            "lib_sha16": _sha16_files([os.path.join(pdir, "libmfft.so")]),
            "commit": commit,
            # the library's own build record: the commit it was built at (this
            # run may have no git metadata) and whether its sources are these
            "build_commit": built.get("commit"), "build_dirty": built.get("dirty"),
            "build_matches_csrc": (built.get("csrc_sha16") == csrc) if built else None}


def compact_line(full: dict, detail: "str | None" = None) -> dict:
    """The driver's line, built from the full record: the contract keys,
    ``roofline`` and ``cpu_baseline``, the N=2048 B=1 latencies, per-size
    ``[N, GB/s, frac]`` triples (real: ``[N, r2c GB/s, r2c frac, c2r GB/s,
    c2r frac]``), configs 2-4 as ``[N, B, api p50 ms, kernel ms]`` rows,
    a summary of config 5, and the provenance hashes.  The per-launch lists,
    vendor columns and config-5 cells stay in the detail record."""
    line = {k: full.get(k) for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                                     "higher_is_better", "scaling", "vs_baseline", "dtype", "data")}
    cfg = full.get("config") or {}
    line["config"] = {k: cfg.get(k) for k in ("workload", "frac_hbm_of_value", "stream_copy_gbps",
                                              "frac_of_stream_copy", "d2d_copy_gbps")}
    if cfg.get("runner_forced"):
        line["config"]["runner_forced"] = cfg["runner_forced"]
    r = full.get("roofline")
    if r:
        line["roofline"] = {k: r.get(k) for k in (
            "bound", "achieved", "peak", "unit", "frac", "traffic", "traffic_over_algorithmic", "kernel",
            "launch_ms", "algorithmic_bytes_per_execute", "copy_ceiling_gbps", "round_trips",
            "frac_of_copy_bound")}
    else:
        line["roofline"] = None
    c = full.get("cpu_baseline")
    if c:
        mt = c.get("all_cores") or {}
        line["cpu_baseline"] = {"value": c.get("value"), "unit": c.get("unit"), "cores": c.get("cores"),
                                "kind": c.get("kind"), "sample": c.get("sample"),
                                "gpu_over_cpu": c.get("gpu_over_cpu"), "cpu_model": c.get("cpu_model"),
                                "all_cores": {"value": mt.get("value"), "cores": mt.get("cores")}}
    else:
        line["cpu_baseline"] = None
    lat = full.get("latency_n2048_b1")
    line["latency_n2048_b1"] = ({k: lat.get(k) for k in (
        "executed", "api_wall_p50_ms", "api_wall_mad_ms", "trials", "kernel_event_p50_ms",
        "graph_replay_us_per_transform", "api_p50_speedup_vs_reference_p800")} if lat else None)
    line["per_size"] = [[p["n"], p["gbps"], p["frac_hbm"]] for p in full.get("per_size") or []]
    real = {}
    for p in full.get("real_per_size") or []:
        real.setdefault(p["n"], {})[p["transform"]] = p
    line["real_per_size"] = [[n, d.get("r2c", {}).get("gbps"), d.get("r2c", {}).get("frac_hbm"),
                              d.get("c2r", {}).get("gbps"), d.get("c2r", {}).get("frac_hbm")]
                             for n, d in sorted(real.items())]
    for key in ("config2", "config4"):
        line[key] = [[c["n"], c["batch"], c["api_wall_p50_ms"], c["kernel_event_p50_ms"]]
                     for c in full.get(key) or []]
    line["config3"] = [[c["n"], c["batch"], c["transform"], c["api_wall_p50_ms"], c["kernel_event_p50_ms"]]
                       for c in full.get("config3") or []]
    cells = full.get("config5") or []
    if cells:
        sp = sorted(c["speedup_vs_m0"] for c in cells)
        mf = sorted(c["mfma_over_selected"] for c in cells)
        line["config5"] = {"cells": len(cells), "clears_guard": sum(bool(c["clears_guard"]) for c in cells),
                           "speedup_vs_m0_min": sp[0], "speedup_vs_m0_median": sp[len(sp) // 2],
                           "speedup_vs_m0_max": sp[-1], "mfma_over_selected_min": mf[0]}
    else:
        line["config5"] = None
    line["provenance"] = full.get("provenance")
    line["detail"] = detail
    # never outgrow the tail the driver reads: shed the least important rows
    for key in ("config3", "config2", "config4"):
        if len(json.dumps(line)) < LINE_LIMIT:
            break
        line[key] = "in detail record"
    return line


def p50_mad(xs):
    """Pooled p50 and median absolute deviation of trial times, both as the
    upper median (the element at len // 2 of the sorted list), the
    reference holdout's convention (scripts/issue10_wp3_holdout.py:510-520)."""
    ys = sorted(xs)
    p50 = ys[len(ys) // 2]
    dev = sorted(abs(v - p50) for v in ys)
    return p50, dev[len(dev) // 2]


def batch_for(n: int) -> int:
    return max(64, (1 << 25) // n)


def real_batch_for(n: int) -> int:
    """R2C/C2R rows: twice the C2C batch, the same bytes per launch (a
    real row moves 4N + 8(N/2+1) bytes, about half of a complex row's 16N),
    so that both transforms are compared at one launch size and working set."""
    return 2 * batch_for(n)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-latency", action="store_true", help="skip the latency / config-2 / config-4 legs")
    ap.add_argument("--no-vendor", action="store_true", help="skip the torch.fft (rocFFT) comparison column")
    ap.add_argument("--sizes", default="", help="comma-separated subset of N (profiling runs)")
    ap.add_argument("--no-real", action="store_true", help="skip the R2C / C2R throughput leg")
    ap.add_argument("--no-config5", action="store_true", help="skip the config-5 selector-vs-M0 sweep")
    ap.add_argument("--runner", default="", help="run every size through this runner name (e.g. "
                    "fft_dit_matrix_batch) instead of the selected plan: profiling runs of one flow")
    ap.add_argument("--detail-out", default=DEFAULT_DETAIL,
                    help="write the full record (per-launch times, vendor columns, config 2-5 cells), "
                         "indented, to this file ('' for none); stdout carries the compact line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: every box here has one MI355X; "
                                   "the batch would shard across GPUs with no exchange, "
                                   "but multi-GPU runs are not part of this benchmark",
                          "n_gpus": args.gpus}))
        return 2

    import numpy as np
    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    from kunlunxin_fft_amd import native, runner
    from kunlunxin_fft_amd.entry import _resolve

    if not torch.cuda.is_available():
        log("bench.py needs a ROCm GPU")
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(0)
    prof = pkg.DeviceProfile.load().hash()
    gen = torch.Generator(device=dev)
    gen.manual_seed(102026)

    sizes = [int(v) for v in args.sizes.split(",") if v] if args.sizes else SIZES

    # ---- device-to-device copy of 256 MiB: the measured bandwidth ceiling
    src = torch.empty(1 << 25, dtype=torch.complex64, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    evs = []
    for _ in range(10):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        dst.copy_(src)
        e.record()
        evs.append((s, e))
    torch.cuda.synchronize()
    copy_ms = statistics.median(s.elapsed_time(e) for s, e in evs)
    copy_gbps = 2 * src.numel() * 8 / (copy_ms * 1e-3) / 1e9
    log(f"d2d copy 256 MiB: {copy_ms:.4f} ms, {copy_gbps:.1f} GB/s (read + write)")

    # ---- the library's streaming copy (non-temporal 16-byte lanes) of 256 MiB
    # each way, each timed copy right after an untimed one of two other
    # buffers so that the MALL holds none of its lines: what a transform that
    # reads and writes every byte once could reach on this device
    src2, dst2 = torch.empty_like(src), torch.empty_like(src)
    nbytes = src.numel() * 8
    sc = torch.cuda.current_stream(dev).cuda_stream
    cevs = []
    for i in range(23):
        native.stream_copy(src2.data_ptr(), dst2.data_ptr(), nbytes, sc)
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        native.stream_copy(src.data_ptr(), dst.data_ptr(), nbytes, sc)
        e.record()
        if i >= 3:
            cevs.append((s, e))
    torch.cuda.synchronize()
    ceil_ms = statistics.median(s.elapsed_time(e) for s, e in cevs)
    ceil_gbps = 2 * nbytes / (ceil_ms * 1e-3) / 1e9
    log(f"streaming copy 256 MiB (flushed): {ceil_ms:.4f} ms, {ceil_gbps:.1f} GB/s (read + write)")
    del src, dst, src2, dst2

    # ---- inputs resident in HBM, plans resolved once (plan reuse)
    work = []
    for n in sizes:
        b = batch_for(n)
        x = torch.randn((b, n), dtype=torch.complex64, device=dev, generator=gen) * math.sqrt(2.0)
        if args.runner:
            plan = pkg.ExecutionPlan(n=n, batch=b, direction="dit", precision="fp32", selection_source="table",
                                     reason="bench.py --runner", fallback=False, executed=args.runner, block=256,
                                     flow_id="bench", flow_realization="bench", processing_unit="bench", params={})
        else:
            plan = pkg.plan_fft("dit", n, batch=b, profile_hash=prof)
        work.append((n, b, x, plan))
        log(f"size N={n} B={b} executed={plan.executed} fallback={plan.fallback}")
    torch.cuda.synchronize()

    def step():
        for _, _, x, plan in work:
            pkg.execute_fft_plan(plan, x)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # A full cyclic-GC pass over torch's object graph stalls the host for tens
    # of milliseconds and leaves the GPU idle; collect and freeze the heap
    # first and keep the collector off while the steps are timed.
    gc.collect()
    gc.freeze()
    gc.disable()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    gc.enable()
    step_bytes = sum(16 * n * b for n, b, _, _ in work)
    wall = t1 - t0
    value = step_bytes * args.steps / wall / 1e9
    ms_per_step = wall / args.steps * 1e3
    log(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step, {value:.1f} GB/s")

    # ---- per size: event time of one execute, and per-launch durations.
    # Measured in the step's own cyclic order, never as back-to-back repeats
    # of one size: repeats rewrite the same 256 MiB output, which then stays
    # in the 256 MB MALL and absorbs the writes (a row copy repeated that way
    # reads 8.3 TB/s, above the HBM peak).  In the cycle, every size starts
    # after the others' traffic, as in the timed steps.
    per_size = []
    stream = torch.cuda.current_stream(dev)
    natives = []
    for n, b, x, plan in work:
        nplan, (shape, dt) = _resolve(plan, 0)
        natives.append((nplan, torch.empty(shape, dtype=dt, device=dev), runner.workspace_for(nplan, dev)))

    def run_native(nplan, x, out, ws):
        nplan.execute_ws(x.data_ptr(), out.data_ptr(), ws.data_ptr() if ws is not None else 0,
                         nplan.ws_bytes, stream.cuda_stream)

    # 100 cycles (each size's median over 100 executes; the timed steps
    # before them are the warm-up)
    evs = [[] for _ in work]
    for _ in range(100):
        for i, (n, b, x, plan) in enumerate(work):
            nplan, out, ws = natives[i]
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record(stream)
            run_native(nplan, x, out, ws)
            e.record(stream)
            evs[i].append((s, e))
    torch.cuda.synchronize()
    # per-launch events: the cyclic predecessor runs first, untimed, so the
    # GPU is busy when the timed launches are queued (no host enqueue gap in
    # the first timed interval) and the caches hold other sizes' data
    launch_runs = [[] for _ in work]
    for _ in range(20):
        for i, (n, b, x, plan) in enumerate(work):
            pn, pout, pws = natives[i - 1]
            run_native(pn, work[i - 1][2], pout, pws)
            nplan, out, ws = natives[i]
            launch_runs[i].append(nplan.execute_timed(x.data_ptr(), out.data_ptr(), stream.cuda_stream,
                                                      ws_ptr=ws.data_ptr() if ws is not None else 0,
                                                      ws_bytes=nplan.ws_bytes))
    def round_trips(flow, launches):
        """HBM round trips of the data in one execute: one for the single-pass
        kernels, two for the four-step (its intermediate Z goes out and back),
        one per launch for the stage flows."""
        if flow in ("lds-fused", "dense-mfma"):
            return 1
        if flow == "four-step":
            return 2
        return launches

    flows = []  # per size: (launch names, per-launch ms) of one execute
    for i, (n, b, x, plan) in enumerate(work):
        nplan, out, _ = natives[i]
        ms = statistics.median(s.elapsed_time(e) for s, e in evs[i])
        per_launch = [statistics.median(col) for col in zip(*launch_runs[i])]
        flow = nplan.flow_name
        rows = int(nplan.info.chunk_rows) or b
        names = []
        for j, t in enumerate(per_launch):
            if flow == "four-step":
                names.append(f"fourstep_pass_kernel pass {j % 2 + 1} "
                             f"(n{'12'[j % 2]}={nplan.info.n1 if j % 2 == 0 else nplan.info.n2})")
            elif flow == "lds-fused":
                names.append("lds_fft_kernel")
            elif flow == "dense-mfma":
                names.append("mfma_fft_kernel")
            else:
                names.append(f"{flow} stage {j + 1}")
        flows.append((names, per_launch, rows))
        gbps = 16 * n * b / (ms * 1e-3) / 1e9
        trips = round_trips(flow, len(per_launch))
        per_size.append({
            "n": n, "batch": b, "executed": plan.executed, "flow": flow,
            "fallback": plan.fallback, "launches": len(per_launch),
            "ms": round(ms, 5), "gbps": round(gbps, 1), "frac_hbm": round(gbps / PEAK_GBPS, 4),
            "gflops": round(5 * n * math.log2(n) * b / (ms * 1e-3) / 1e9, 1),
            "launch_ms": [round(t, 5) for t in per_launch],
            "split": [int(nplan.info.n1), int(nplan.info.n2), rows] if nplan.info.n1 else None,
            "round_trips": trips, "frac_of_copy_bound": round(gbps * trips / ceil_gbps, 4),
        })
        log(f"N={n:>8} B={b:>6} {flow:>10} {ms:8.4f} ms {gbps:8.1f} GB/s "
            f"({gbps / PEAK_GBPS:.1%}) launches={['%.4f' % t for t in per_launch]}")

    # ---- dominant kernel: the size whose launches take the most time per step.
    # A flow of several launches (the four-step's two passes, per chunk) is
    # one unit: the transforms' algorithmic bytes (16 N per row, read once and
    # written once) over the sum of all launch durations of one execute.
    di = max(range(len(work)), key=lambda i: sum(flows[i][1]))
    dn, db = work[di][0], work[di][1]
    dnames, dts, drows = flows[di]
    dflow = natives[di][0].flow_name
    d_bytes = 16 * dn * db
    d_ms = sum(dts)
    d_ach = d_bytes / (d_ms * 1e-3) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    if os.path.exists(tpath):
        try:
            tmap = json.load(open(tpath))
            parts = [tmap.get(f"{nm}|N={dn}|rows={drows}") for nm in dnames]
            traffic = sum(parts) if all(v is not None for v in parts) else None
        except (OSError, ValueError, TypeError):
            traffic = None
    kinds = sorted(set(dnames), key=dnames.index)
    roofline = {"bound": "hbm", "achieved": round(d_ach, 1), "peak": PEAK_GBPS, "unit": "GB/s",
                "frac": round(d_ach / PEAK_GBPS, 4), "traffic": traffic,
                "traffic_over_algorithmic": round(traffic / d_bytes, 3) if traffic else None,
                "kernel": f"{' + '.join(kinds)} [{dflow}, N={dn}, B={db}, {drows} rows per launch, "
                          f"{len(dts)} launches per execute, counted together]",
                "algorithmic_bytes_per_execute": d_bytes, "launch_ms": [round(t, 5) for t in dts],
                "sum_launch_ms": round(d_ms, 5), "share_of_step": round(d_ms / ms_per_step, 3),
                "copy_ceiling_gbps": round(ceil_gbps, 1), "round_trips": round_trips(dflow, len(dts)),
                "frac_of_copy_bound": round(d_ach * round_trips(dflow, len(dts)) / ceil_gbps, 4)}
    log(f"dominant kernel: {roofline}")

    # ---- latency at N=2048 B=1 (reference protocol) and config 2
    def latency(n, b, ttype="c2c", tdir=None):
        rng = np.random.default_rng(102026 + 10 * n + b)
        m = n // 2 + 1 if ttype == "c2r" else n
        if ttype == "r2c":
            h = rng.standard_normal((b, n)).astype(np.float32)
            nbytes = b * (4 * n + 8 * (n // 2 + 1))
        else:
            h = (rng.standard_normal((b, m)) + 1j * rng.standard_normal((b, m))).astype(np.complex64)
            nbytes = b * (4 * n + 8 * (n // 2 + 1)) if ttype == "c2r" else 16 * n * b
        x = torch.from_numpy(h[0] if b == 1 else h).to(dev)
        plan = pkg.plan_fft("dit", n, batch=b, profile_hash=prof, transform_type=ttype,
                            transform_direction=tdir)
        for _ in range(5):
            pkg.execute_fft_plan(plan, x)
        torch.cuda.synchronize()
        wall = []
        for _ in range(5):
            for _ in range(32):
                a = time.perf_counter()
                pkg.execute_fft_plan(plan, x)
                torch.cuda.synchronize()
                wall.append((time.perf_counter() - a) * 1e3)
        nplan, (shape, dt) = _resolve(plan, 0)
        out = torch.empty(shape, dtype=dt, device=dev)
        ws = runner.workspace_for(nplan, dev)
        evs = []
        for _ in range(100):
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record(stream)
            run_native(nplan, x, out, ws)
            e.record(stream)
            evs.append((s, e))
        torch.cuda.synchronize()
        ev = statistics.median(s.elapsed_time(e) for s, e in evs)
        p50, mad = p50_mad(wall)
        return {"n": n, "batch": b, "transform": f"{ttype} {plan.transform_direction}",
                "executed": plan.executed, "api_wall_p50_ms": round(p50, 5), "api_wall_mad_ms": round(mad, 5),
                "trials": len(wall), "kernel_event_p50_ms": round(ev, 5),
                "api_gbps": round(nbytes / (p50 * 1e-3) / 1e9, 3),
                "kernel_gbps": round(nbytes / (ev * 1e-3) / 1e9, 1)}

    def graph_replay_us(n, reps_per_graph=64, replays=20):
        """Per-transform time of N-point B=1 executes recorded into one HIP
        graph (torch.cuda.CUDAGraph) and replayed: what a launch-bound caller
        gets without the per-call host path."""
        plan = pkg.plan_fft("dit", n, batch=1, profile_hash=prof)
        x = torch.randn((n,), dtype=torch.complex64, device=dev, generator=gen)
        pkg.execute_fft_plan(plan, x)
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            pkg.execute_fft_plan(plan, x)
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=side):
                for _ in range(reps_per_graph):
                    pkg.execute_fft_plan(plan, x)
        torch.cuda.synchronize()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(replays):
            graph.replay()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / (replays * reps_per_graph) * 1e6

    lat, cfg2, cfg3, cfg4 = None, [], [], []
    if not args.no_latency:
        lat = latency(2048, 1)
        lat["graph_replay_us_per_transform"] = round(graph_replay_us(2048), 3)
        # the reference's published p50 for this cell on its own hardware (Kunlunxin P800,
        # frozen selector, results/p800/issue9_v61/reports/steady_report.csv:55); context only
        lat["reference_p800_api_p50_ms"] = 0.4036
        lat["api_p50_speedup_vs_reference_p800"] = round(0.4036 / lat["api_wall_p50_ms"], 1)
        log(f"latency N=2048 B=1: {lat}")
        cfg2 = [latency(n, b) for n in (1024, 2048) for b in (16, 64)]
        for c in cfg2:
            log(f"config2: {c}")
        # config 3: inverse C2C and the real pair at N in {256, 4096}, B in {1, 64}
        cfg3 = [latency(n, b, t, d) for n in (256, 4096) for b in (1, 64)
                for t, d in (("c2c", "inverse"), ("r2c", "forward"), ("c2r", "inverse"))]
        for c in cfg3:
            log(f"config3: {c}")
        cfg4 = [latency(1 << 20, 1), latency(1 << 16, 256)]
        for c in cfg4:
            log(f"config4: {c}")

    # ---- R2C and C2R throughput at the same sizes (selected plans), twice
    # the C2C batch so that a launch moves the same bytes as the C2C row
    # (algorithmic bytes per row are 4N (real side) + 8(N/2+1) (half
    # spectrum), about half of C2C's 16N), timed in cyclic order like per_size
    real_rows = []
    if not args.no_real:
        rwork = []
        for n in sizes:
            b = real_batch_for(n)
            xr = torch.randn((b, n), dtype=torch.float32, device=dev, generator=gen)
            xc = torch.randn((b, n // 2 + 1), dtype=torch.complex64, device=dev, generator=gen)
            for tt, td, x in (("r2c", "forward", xr), ("c2r", "inverse", xc)):
                plan = pkg.plan_fft("dit", n, batch=b, profile_hash=prof, transform_type=tt, transform_direction=td)
                nplan, (shape, dt) = _resolve(plan, 0)
                rwork.append((n, b, tt, x, plan, nplan, torch.empty(shape, dtype=dt, device=dev),
                              runner.workspace_for(nplan, dev)))
        for _, _, _, x, _, nplan, out, ws in rwork:
            run_native(nplan, x, out, ws)
        revs = [[] for _ in rwork]
        for _ in range(5):
            for i, (_, _, _, x, _, nplan, out, ws) in enumerate(rwork):
                s = torch.cuda.Event(enable_timing=True)
                e = torch.cuda.Event(enable_timing=True)
                s.record(stream)
                run_native(nplan, x, out, ws)
                e.record(stream)
                revs[i].append((s, e))
        torch.cuda.synchronize()
        for i, (n, b, tt, _, plan, nplan, _, _) in enumerate(rwork):
            ms = statistics.median(s.elapsed_time(e) for s, e in revs[i])
            gbps = b * (4 * n + 8 * (n // 2 + 1)) / (ms * 1e-3) / 1e9
            real_rows.append({"n": n, "batch": b, "transform": tt, "executed": plan.executed,
                              "fallback": plan.fallback, "flow": nplan.flow_name, "launches": int(nplan.info.launches), "ms": round(ms, 5),
                              "gbps": round(gbps, 1), "frac_hbm": round(gbps / PEAK_GBPS, 4),
                              "split": ([int(nplan.info.n1), int(nplan.info.n2), int(nplan.info.chunk_rows) or b]
                                        if nplan.info.n1 else None)})
            log(f"{tt} N={n:>8} B={b:>6} {nplan.flow_name:>10} {ms:8.4f} ms {gbps:8.1f} GB/s "
                f"({gbps / PEAK_GBPS:.1%}) launches={nplan.info.launches}")
        del rwork

    # ---- vendor comparison column: rocFFT through torch.fft on the same inputs
    if not args.no_vendor:
        for (n, b, x, plan), row in zip(work, per_size):
            for _ in range(3):
                torch.fft.fft(x, dim=-1)
            evs = []
            for _ in range(10):
                s = torch.cuda.Event(enable_timing=True)
                e = torch.cuda.Event(enable_timing=True)
                s.record(stream)
                torch.fft.fft(x, dim=-1)
                e.record(stream)
                evs.append((s, e))
            torch.cuda.synchronize()
            vms = statistics.median(s.elapsed_time(e) for s, e in evs)
            row["vendor_ms"] = round(vms, 5)
            row["vendor_gbps"] = round(16 * n * b / (vms * 1e-3) / 1e9, 1)
            log(f"N={n:>8} B={b:>6} torch.fft (rocFFT) {vms:8.4f} ms {row['vendor_gbps']:8.1f} GB/s "
                f"(this library {row['ms']:.4f} ms)")

    # ---- config 5: the selector sweep, N = 16 .. 2^14 x B in {1, 16, 64, 256},
    # forward C2C.  Per cell: the selected plan and the M0 incumbent (fft_dit /
    # fft_dit_batch), each timed as the table builder times a cell (20
    # back-to-back executes replayed from a HIP graph between HIP events,
    # median of 5 replays: device time, since a host loop of enqueues would
    # time the host in these launch-bound cells), and whether the selected
    # plan still clears the reference's 2% promotion guard
    # (src/xpu/selector.py:59-63) in this run.
    cfg5 = []
    if not args.no_config5:
        from kunlunxin_fft_amd.selector import GUARD_PCT as guard

        def cell_ms(plan, x, reps=20, rounds=5):
            nplan, (shape, dt) = _resolve(plan, 0)
            out = torch.empty(shape, dtype=dt, device=dev)
            ws = runner.workspace_for(nplan, dev)
            return runner.time_native_graph(nplan, x, out, ws, reps=reps, rounds=rounds), nplan.flow_name

        for n in [1 << k for k in range(4, 15)]:
            for b in (1, 16, 64, 256):
                x = torch.randn((n,) if b == 1 else (b, n), dtype=torch.complex64, device=dev, generator=gen)
                sel = pkg.plan_fft("dit", n, batch=b, profile_hash=prof)
                m0 = pkg.plan_fft("dit", n, batch=b)  # no profile: the M0 closure
                # the dense-dot MFMA candidate (the reference's M2 flow) in every cell
                mname = "fft_dit_matrix" + ("_batch" if b > 1 else "")
                mf = pkg.ExecutionPlan(n=n, batch=b, direction="dit", precision="fp32", selection_source="table",
                                       reason="bench.py config-5 MFMA candidate", fallback=False, executed=mname,
                                       block=256, flow_id="bench", flow_realization="bench",
                                       processing_unit="bench", params={})
                sel_ms, sel_flow = cell_ms(sel, x)
                m0_ms, _ = cell_ms(m0, x)
                mf_ms, mf_flow = cell_ms(mf, x)
                row = {"n": n, "batch": b, "selected": sel.executed, "selected_flow": sel_flow,
                       "selection_source": sel.selection_source, "selected_us": round(sel_ms * 1e3, 2),
                       "m0": m0.executed, "m0_us": round(m0_ms * 1e3, 2),
                       "speedup_vs_m0": round(m0_ms / sel_ms, 2),
                       "mfma_candidate": mname, "mfma_flow": mf_flow, "mfma_us": round(mf_ms * 1e3, 2),
                       "mfma_over_selected": round(mf_ms / sel_ms, 2),
                       "guard_pct": guard, "clears_guard": bool(sel_ms <= m0_ms * (1 - guard / 100.0))}
                cfg5.append(row)
                log(f"config5 N={n:>6} B={b:>4} {sel.executed:>22} {row['selected_us']:8.2f} us "
                    f"M0 {row['m0_us']:8.2f} us  x{row['speedup_vs_m0']:.2f} guard={'ok' if row['clears_guard'] else 'NO'}"
                    f"  MFMA {row['mfma_us']:8.2f} us")
                del x
        torch.cuda.synchronize()

    # ---- CPU baseline (reference CPU path, 1 core, bounded sample)
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle  # the reference CPU path / its restatement, timed as the baseline

        rng = np.random.default_rng(7)
        rows = 16  # per size: a batch of 16 transforms of each N
        threads = max(1, min(16, os.cpu_count() or 1))
        tot_s, tot_mt, tot_bytes, kinds = 0.0, 0.0, 0, set()
        for n in SIZES:
            h = rng.standard_normal((rows, n)) + 1j * rng.standard_normal((rows, n))
            s, kind = oracle.time_cpu_fft(h, threads=1, reps=5)
            kinds.add(kind)
            tot_s += s
            s_mt, kind_mt = oracle.time_cpu_fft(h, threads=threads, reps=5)
            kinds.add(kind_mt)
            tot_mt += s_mt
            tot_bytes += 16 * n * rows
        # the first processor's identity: a virtual machine's model name can
        # be as short as "AMD EPYC", so vendor, family, model and clock too
        info = {}
        try:
            for ln in open("/proc/cpuinfo"):
                if not ln.strip():
                    break
                k, _, v = ln.partition(":")
                info.setdefault(k.strip(), v.strip())
        except OSError:
            pass
        model = info.get("model name", "unknown")
        cpu_id = " ".join(f"{k} {info[k]}" for k in ("vendor_id", "cpu family", "model", "stepping", "cpu MHz")
                          if k in info)
        try:
            usable = len(os.sched_getaffinity(0))
        except (AttributeError, OSError):
            usable = os.cpu_count() or 1
        cpu = {"value": round(tot_bytes / tot_s / 1e9, 4), "unit": "GB/s", "cores": 1,
               "cpu_model": model, "cpu_id": cpu_id, "host_cpus": os.cpu_count(), "usable_cpus": usable,
               "kind": "reference" if kinds == {"reference"} else "port",
               "sample": f"{rows} transforms of each N = 2^10..2^20 (complex<double>, butterfly::fft_dit "
                         f"with its per-stage twiddle rebuild), median of 5 passes, {tot_s:.1f} s per pass",
               "gpu_over_cpu": round(value / (tot_bytes / tot_s / 1e9), 1),
               "all_cores": {"value": round(tot_bytes / tot_mt / 1e9, 4), "cores": threads,
                             "sample": f"the same rows split over {threads} std::threads "
                                       f"(host reports {os.cpu_count()} CPUs), {tot_mt:.2f} s per pass"}}
        log(f"cpu baseline: {cpu}")

    full = {
        "metric": METRIC,
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "complex64 (fp32)",
        "data": "synthetic: iid N(0,1) real/imag parts, fixed device seed, resident in HBM",
        "config": {"workload": WORKLOAD,
                   "frac_hbm_of_value": round(value / PEAK_GBPS, 4),
                   "runner_forced": args.runner or None,
                   "d2d_copy_gbps": round(copy_gbps, 1),
                   "frac_of_d2d_copy": round(value / copy_gbps, 4),
                   "stream_copy_gbps": round(ceil_gbps, 1),
                   "frac_of_stream_copy": round(value / ceil_gbps, 4)},
        "provenance": provenance(pkg, prof),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "latency_n2048_b1": lat,
        "config2": cfg2,
        "config3": cfg3,
        "config4": cfg4,
        "config5": cfg5,
        "per_size": per_size,
        "real_per_size": real_rows,
    }
    detail = args.detail_out
    if detail:
        try:
            os.makedirs(os.path.dirname(os.path.abspath(detail)), exist_ok=True)
            with open(detail, "w") as f:
                json.dump(full, f, indent=1)
        except OSError as e:
            log(f"detail record not written ({detail}): {e}")
            detail = ""
    # the one line the driver parses: last on stdout, a few KB at most
    print(json.dumps(compact_line(full, os.path.relpath(detail, ROOT) if detail else None)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
