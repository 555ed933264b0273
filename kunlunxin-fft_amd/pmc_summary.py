"""Profile summaries for bench.py runs under rocprofv3 (CSV output).

``traffic``: HBM traffic per kernel launch from two ``rocprofv3 --pmc`` runs.

Reads the counter CSVs of a FETCH_SIZE run and a WRITE_SIZE run (counter
values in KiB per dispatch, ``--output-format csv``), averages them per
(kernel, grid), scales each counter by what it reads for the device copy of
known size that bench.py performs first (256 MiB read + 256 MiB written,
kernel ``__amd_rocclr_copyBuffer``), and matches every FFT kernel to the
bench.py size it belongs to using the ``bench_detail.json`` that the same
bench.py command writes: a dispatch of ``grid`` threads with 2^LOGE elements
per thread covers grid * 2^LOGE complex points.

Writes
  * a JSON map ``"<kernel as bench.py names it>|N=<n>|rows=<rows per launch>"
    -> HBM bytes per launch``, which bench.py reports as ``roofline.traffic``;
  * a Markdown table (algorithmic bytes, measured bytes, their ratio).

``stats``: kernel durations per launch shape (kernel, grid) from the
kernel_trace.csv of ``rocprofv3 --kernel-trace``, as Markdown.

Usage:
    python kunlunxin-fft_amd/pmc_summary.py traffic --fetch DIR --write DIR --detail bench_detail.json \
        --json profiles/pmc_traffic.json --md profiles/<name>.md [--sq DIR] [--trace DIR] [--command TEXT]
    python kunlunxin-fft_amd/pmc_summary.py stats --dir DIR --md profiles/<name>.md [--detail bench_detail.json] [--command TEXT]
"""
from __future__ import annotations

import argparse
import collections
import csv
import glob
import json
import os
import re
import sys

COPY_KERNEL = "__amd_rocclr_copyBuffer"
COPY_BYTES = 256 << 20  # bench.py's calibration copy: 256 MiB each way


def _counter_rows(d: str):
    files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {d}")
    for path in files:
        with open(path, newline="") as f:
            yield from csv.DictReader(f)


def _short(name: str) -> str:
    """Kernel symbol without return type, namespaces and parameter list."""
    name = name.replace("void ", "").replace("mfft::(anonymous namespace)::", "")
    return re.sub(r"\(.*$", "", name)


def _template_args(name: str):
    m = re.search(r"<([^<>]*)>", name)
    if not m:
        return None
    try:
        return [int(t.strip()) for t in m.group(1).split(",")]
    except ValueError:
        return None


def per_kernel(d: str, counter: str):
    acc = collections.defaultdict(list)
    for r in _counter_rows(d):
        if r.get("Counter_Name") != counter:
            continue
        name = _short(r["Kernel_Name"])
        acc[(name, int(r["Grid_Size"]))].append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in acc.items()}


def bench_keys(name: str, grid: int, sizes) -> list:
    """bench.py kernel keys ("<kernel>|N=<n>|rows=<rows per launch>") that a
    dispatch of ``name`` over ``grid`` threads serves; a dispatch of grid
    threads with 2^LOGE elements per thread covers grid * 2^LOGE points.
    Two sizes can share one (kernel, grid), e.g. pass 2 of 2^19 and 2^20
    points.  Persistent kernels are not matched: their grid is the resident
    wave, not the work."""
    t = _template_args(name)
    if t is None or not name.startswith(("fourstep_pass_kernel", "lds_fft_kernel")):
        return []
    logl, loge = t[0], t[1]
    points = grid << loge
    keys = []
    for s in sizes:
        n = s["n"]
        if name.startswith("lds_fft_kernel") and s["flow"] == "lds-fused" and n == (1 << logl):
            if points == n * s["batch"]:  # one launch per execute covers the batch
                keys.append(f"lds_fft_kernel|N={n}|rows={points // n}")
        elif name.startswith("fourstep") and s["flow"] == "four-step" and s.get("split"):
            n1, n2, rows = s["split"]
            kind = t[4]
            # the bench's C2C rows are forward transforms (DIR -1)
            if rows * n == points and (n1 if kind == 0 else n2) == (1 << logl) and t[3] == -1:
                keys.append(f"fourstep_pass_kernel pass {kind + 1} (n{kind + 1}={1 << logl})"
                            f"|N={n}|rows={rows}")
    return keys


def real_keys(name: str, grid: int, real_sizes) -> list:
    """Labels ("<transform> <kernel>|N=<n>|rows=<rows>") for the launches of
    bench.py's real-transform leg (``real_per_size``): the LDS kernel's R2C
    (mode 1) and C2R (mode 2) instances, the four-step passes over the
    half-length core, and the standalone stitch / pre-twiddle kernels (one
    thread per mirror pair, 256-thread blocks per row)."""
    keys = []
    t = _template_args(name)
    for s in real_sizes:
        n, b, tt = s["n"], s["batch"], s["transform"]
        core = n // 2
        if name.startswith("lds_fft_kernel") and t is not None and len(t) == 4 and s["flow"] == "lds-fused":
            logl, loge, mode = t[0], t[1], t[3]
            if (mode, tt) in ((1, "r2c"), (2, "c2r")) and core == (1 << logl) and (grid << loge) == core * b:
                keys.append(f"{tt} lds_fft_kernel|N={n}|rows={b}")
        elif name.startswith("fourstep_pass_kernel") and t is not None and s["flow"] == "four-step" and s.get("split"):
            n1, n2, rows = s["split"]
            logl, loge, kind = t[0], t[1], t[4]
            # r2c runs a forward core (DIR -1), c2r an inverse one (DIR +1)
            if (rows * core == (grid << loge) and (n1 if kind == 0 else n2) == (1 << logl)
                    and t[3] == (-1 if tt == "r2c" else 1)):
                keys.append(f"{tt} pass {kind + 1}|N={n}|rows={rows}")
        elif name.startswith(("r2c_stitch_kernel", "c2r_pre_kernel")) and s["flow"] == "four-step":
            want = "r2c" if name.startswith("r2c") else "c2r"
            bpr = ((core >> 1) + 1 + 255) // 256
            if tt == want and grid == bpr * b * 256:
                keys.append(f"{tt} {name}|N={n}|rows={b}")
    return keys


SQ_COUNTERS = ("SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_INSTS_LDS", "SQ_INSTS_VALU")


def calibration(d: str, counter: str) -> float:
    """Counter KiB per KiB actually moved, from bench.py's 256 MiB copies.

    Those are the device copies dispatched before the first other kernel of
    the run; later copies (inputs, vendor comparisons) have other sizes.
    """
    rows = sorted((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"]))
                  for r in _counter_rows(d) if r.get("Counter_Name") == counter)
    vals = []
    for _, name, v in rows:
        if not name.startswith(COPY_KERNEL):
            break
        vals.append(v)
    if not vals:
        raise SystemExit(f"the {counter} run starts with no device copy to calibrate against")
    vals.sort()
    return vals[len(vals) // 2] / (COPY_BYTES / 1024)


def _commands(f, command: str) -> None:
    if command:
        f.write("Commands (repo root, TMPDIR=/tmp):\n\n")
        for line in command.split(";"):
            f.write(f"    {line.strip()}\n")
        f.write("\n")


def trace_durations(d: str) -> dict:
    """(kernel, grid threads) -> list of dispatch durations in ns, from the
    kernel_trace.csv of a ``rocprofv3 --kernel-trace`` run."""
    files = glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *kernel_trace.csv under {d}")
    durs = collections.defaultdict(list)
    with open(files[0], newline="") as f:
        for r in csv.DictReader(f):
            grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            durs[(_short(r["Kernel_Name"]), grid)].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    return durs


def stats(args) -> int:
    """Per (kernel, grid) durations from kernel_trace.csv: one kernel name
    covers several launch shapes (sizes, chunks), which kernel_stats.csv
    averages together."""
    durs = trace_durations(args.dir)
    detail = json.load(open(args.detail)) if args.detail else {}
    sizes = detail.get("per_size", [])
    real_sizes = detail.get("real_per_size", [])
    total = sum(sum(v) for v in durs.values())
    order = sorted(durs.items(), key=lambda kv: -sum(kv[1]))[: args.top]
    with open(args.md, "w") as f:
        f.write("# Kernel durations per launch shape (rocprofv3 --kernel-trace)\n\n")
        _commands(f, args.command)
        f.write("Rows are (kernel, grid threads) from kernel_trace.csv, the largest total first; "
                "`bench key` names the bench.py size a launch shape serves.\n\n")
        f.write("| kernel | grid | bench key | calls | total ms | average us | min us | max us | share |\n")
        f.write("|---|---:|---|---:|---:|---:|---:|---:|---:|\n")
        for (name, grid), v in order:
            keys = ", ".join([k.split("|", 1)[1] for k in bench_keys(name, grid, sizes)]
                             + [k.split("|", 1)[0].split(" ", 1)[0] + " " + k.split("|", 1)[1]
                                for k in real_keys(name, grid, real_sizes)]) or "-"
            keys = keys.replace("|", "\\|")  # a literal pipe inside a Markdown table cell
            f.write(f"| {name} | {grid} | {keys} | {len(v)} | {sum(v) / 1e6:.3f} | {sum(v) / len(v) / 1e3:.2f} | "
                    f"{min(v) / 1e3:.2f} | {max(v) / 1e3:.2f} | {100.0 * sum(v) / total:.1f}% |\n")
    print(f"wrote {args.md} ({len(order)} launch shapes)")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True, help="output dir of the FETCH_SIZE run")
    t.add_argument("--write", required=True, help="output dir of the WRITE_SIZE run")
    t.add_argument("--detail", required=True, help="bench_detail.json written by the same bench command")
    t.add_argument("--json", required=True)
    t.add_argument("--md", required=True)
    t.add_argument("--command", default="", help="commands that made the input, quoted in the Markdown")
    t.add_argument("--sq", default="", help="output dir of an SQ counter run (" + " ".join(SQ_COUNTERS) + ")")
    t.add_argument("--trace", default="", help="output dir of a --kernel-trace run of the same command (rates)")
    st = sub.add_parser("stats")
    st.add_argument("--dir", required=True, help="output dir of the --kernel-trace --stats run")
    st.add_argument("--md", required=True)
    st.add_argument("--detail", default="", help="bench_detail.json of the same command (labels the rows)")
    st.add_argument("--top", type=int, default=40, help="launch shapes listed")
    st.add_argument("--command", default="")
    args = ap.parse_args()
    if args.cmd == "stats":
        return stats(args)

    fetch = per_kernel(args.fetch, "FETCH_SIZE")
    write = per_kernel(args.write, "WRITE_SIZE")
    f_cal, w_cal = calibration(args.fetch, "FETCH_SIZE"), calibration(args.write, "WRITE_SIZE")
    sq = {c: per_kernel(args.sq, c) for c in SQ_COUNTERS} if args.sq else {}
    durs = trace_durations(args.trace) if args.trace else {}
    sizes = json.load(open(args.detail))["per_size"]

    rows_out, traffic = [], {}
    for (name, grid) in sorted(set(fetch) | set(write)):
        keys = bench_keys(name, grid, sizes)
        if not keys:
            continue
        points = grid << _template_args(name)[1]
        fb = fetch.get((name, grid), float("nan")) * 1024 / f_cal
        wb = write.get((name, grid), float("nan")) * 1024 / w_cal
        alg = 16 * points
        for key in keys:
            traffic[key] = round(fb + wb)
            rows_out.append((key, name, grid, alg, fb, wb))

    with open(args.json, "w") as f:
        json.dump(traffic, f, indent=1, sort_keys=True)
    with open(args.md, "w") as f:
        f.write("# HBM traffic per launch (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE)\n\n")
        _commands(f, args.command)
        f.write(f"Calibration: the 256 MiB device copy ({COPY_KERNEL}) reads FETCH_SIZE = "
                f"{f_cal * 256:.2f} MiB and WRITE_SIZE = {w_cal * 256:.2f} MiB, so FETCH_SIZE is scaled "
                f"by {1 / f_cal:.3f} and WRITE_SIZE by {1 / w_cal:.3f}.  Algorithmic bytes = 16 per point "
                f"(one complex64 read + one written).\n\n")
        if sq:
            f.write("SQ columns (a third run): LDS bank-conflict cycles per LDS-active cycle "
                    "(SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE) and LDS per VALU instructions.\n\n")
        if durs:
            f.write("Rate columns (the kernel-trace run of the same bench command): the measured bytes over the "
                    "average rocprofv3 duration of the same launch shape, and that rate against 8 TB/s.\n\n")
        f.write("| bench kernel key | kernel | grid | algorithmic MiB | fetch MiB | write MiB | traffic / algorithmic |"
                + (" LDS conflict / active | LDS / VALU insts |" if sq else "")
                + (" rocprof avg us | HBM GB/s | % of 8 TB/s |" if durs else "") + "\n")
        f.write("|---|---|---:|---:|---:|---:|---:|" + ("---:|---:|" if sq else "") + ("---:|---:|---:|" if durs else "")
                + "\n")
        for key, name, grid, alg, fb, wb in rows_out:
            extra = ""
            if sq:
                g = lambda c: sq[c].get((name, grid))  # noqa: E731
                bc, act, li, vi = (g(c) for c in SQ_COUNTERS)
                extra = (f" {bc / act:.3f} |" if bc is not None and act else " - |") + \
                        (f" {li / vi:.3f} |" if li is not None and vi else " - |")
            if durs:
                v = durs.get((name, grid))
                if v:
                    us = sum(v) / len(v) / 1e3
                    gbs = (fb + wb) / (us * 1e-6) / 1e9
                    extra += f" {us:.2f} | {gbs:.0f} | {gbs / 8000:.1%} |"
                else:
                    extra += " - | - | - |"
            f.write(f"| {key.replace('|', chr(92) + '|')} | {name} | {grid} | {alg / 2**20:.1f} | {fb / 2**20:.1f} | {wb / 2**20:.1f} | "
                    f"{(fb + wb) / alg:.3f} |{extra}\n")
    print(f"wrote {args.json} ({len(traffic)} kernels) and {args.md}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
