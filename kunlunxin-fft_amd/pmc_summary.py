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

``counters``: matrix-core use per launch shape (MFMA busy fraction and fp32
MFMA TFLOP/s) from ``rocprofv3 --pmc`` runs of the MFMA counters.

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
    """Integer template arguments of a kernel name (``true`` / ``false`` as
    1 / 0), or None."""
    m = re.search(r"<([^<>]*)>", name)
    if not m:
        return None
    out = []
    for t in m.group(1).split(","):
        t = t.strip()
        if t in ("true", "false"):
            out.append(int(t == "true"))
            continue
        try:
            out.append(int(t))
        except ValueError:
            return None
    return out


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
    if t is None or not name.startswith(("fourstep_pass_kernel", "lds_fft_kernel", "mfma_fft_kernel")):
        return []
    if name.startswith("mfma_fft_kernel"):
        # 16 points per thread at every length (4096 or L points per block)
        return [f"mfma_fft_kernel|N={s['n']}|rows={s['batch']}" for s in sizes
                if s["flow"] == "dense-mfma" and s["n"] == (1 << t[0]) and grid * 16 == s["n"] * s["batch"]]
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
    thread per mirror pair over the flat batch, in 256-thread blocks)."""
    keys = []
    t = _template_args(name)
    for s in real_sizes:
        n, b, tt = s["n"], s["batch"], s["transform"]
        core = n // 2
        if name.startswith("lds_fft_kernel") and t is not None and len(t) in (4, 5) and s["flow"] == "lds-fused":
            logl, loge, mode = t[0], t[1], t[3]
            if (mode, tt) in ((1, "r2c"), (2, "c2r")) and core == (1 << logl) and (grid << loge) == core * b:
                keys.append(f"{tt} lds_fft_kernel|N={n}|rows={b}")
        elif name.startswith("fourstep_pass_kernel") and t is not None and s["flow"] == "four-step" and s.get("split"):
            n1, n2, rows = s["split"]
            logl, loge, kind = t[0], t[1], t[4]
            # the plain pass serves one real launch: C2R's pass 2, the
            # inverse (DIR +1) row pass; R2C's passes and C2R's pass 1 are
            # the fused real kernels below
            if (tt == "c2r" and kind == 1 and t[3] == 1 and rows * core == (grid << loge)
                    and n2 == (1 << logl)):
                keys.append(f"{tt} pass 2|N={n}|rows={rows}")
        elif (name.startswith(("fourstep_r2c_pass", "fourstep_c2r_pass")) and t is not None
              and s["flow"] == "four-step" and s.get("split")):
            # the fused real passes: R2C pass 1 / pass 2 (stitch) and C2R
            # pass 1 (pre-twiddle); <LOGL, LOGE, LOGC>, one block per LOGC
            # columns of a row, so grid << LOGE points per launch
            n1, n2, rows = s["split"]
            logl, loge = t[0], t[1]
            want, p = {"fourstep_r2c_pass1_kernel": ("r2c", 1), "fourstep_r2c_pass2_kernel": ("r2c", 2),
                       "fourstep_c2r_pass1_kernel": ("c2r", 1)}[name.split("<")[0]]
            if tt == want and rows * core == (grid << loge) and (n1 if p == 1 else n2) == (1 << logl):
                keys.append(f"{tt} pass {p}|N={n}|rows={rows}")
        elif name.startswith(("r2c_stitch_kernel", "c2r_pre_kernel")) and s["flow"] != "lds-fused":
            # around a non-fused core: once per execute, or once per chunk of
            # a chunked four-step core
            want = "r2c" if name.startswith("r2c") else "c2r"
            pairs = (core >> 1) + 1
            rows = s["split"][2] if s.get("split") else b
            for r in sorted({b, rows}):
                if tt == want and grid == (r * pairs + 255) // 256 * 256:
                    keys.append(f"{tt} {name}|N={n}|rows={r}")
    return keys


def real_alg_bytes(n: int) -> int:
    """Algorithmic bytes of one real-transform row: n float32 one way, n/2+1
    complex64 the other."""
    return 4 * n + 8 * (n // 2 + 1)


def execute_rows(traffic: dict, sizes, real_sizes) -> list:
    """Per size: HBM bytes of all launches of one execute (every launch key
    that size owns, times the launches of that key per execute = batch / rows
    per launch), against the transform's algorithmic bytes."""
    out = []
    for rows_list, alg_row, key_of in (
            (sizes, lambda n: 16 * n, lambda k, s: not k.startswith(("r2c ", "c2r "))),
            (real_sizes, real_alg_bytes, lambda k, s: k.startswith(s["transform"] + " "))):
        for s in rows_list:
            n, b = s["n"], s["batch"]
            mine = [k for k in traffic if f"|N={n}|rows=" in k and key_of(k, s)]
            if not mine:
                continue
            total = sum(traffic[k] * (b // int(k.rsplit("=", 1)[1])) for k in mine)
            alg = alg_row(n) * b
            out.append({"transform": s.get("transform", "c2c"), "n": n, "batch": b, "flow": s["flow"],
                        "launch_keys": sorted(k.split("|", 1)[0] for k in mine),
                        "hbm_bytes": total, "algorithmic_bytes": alg, "ratio": round(total / alg, 3)})
    return out


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


def agent_facts(d: str) -> dict:
    """SIMD and XCD counts of the GPU agent, from run_agent_info.csv."""
    files = glob.glob(os.path.join(d, "**", "*agent_info.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *agent_info.csv under {d}")
    with open(files[0], newline="") as f:
        for r in csv.DictReader(f):
            if r.get("Agent_Type") == "GPU":
                return {"simd": int(r["Simd_Count"]), "xcc": int(r["Num_Xcc"]), "cu": int(r["Cu_Count"])}
    raise SystemExit(f"no GPU agent in {files[0]}")


MFMA_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_F32", "SQ_INSTS_MFMA", "SQ_BUSY_CU_CYCLES",
                 "GRBM_GUI_ACTIVE")


def counters(args) -> int:
    """Matrix-core use per launch shape: MfmaUtil = SQ_VALU_MFMA_BUSY_CYCLES /
    (GRBM_GUI_ACTIVE of one XCD x SIMDs) (the rocprofv3 derived metric; the
    CSV sums GRBM_GUI_ACTIVE over the XCDs), and fp32 MFMA TFLOP/s = 512 x
    SQ_INSTS_VALU_MFMA_MOPS_F32 over the launch shape's average duration in a
    kernel-trace run of the same command."""
    with open(args.md, "w") as f:
        f.write("# Matrix-core use per launch (rocprofv3 --pmc " + " ".join(MFMA_COUNTERS) + ")\n\n")
        _commands(f, args.command)
        f.write("MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD x SIMDs), rocprofv3's MfmaUtil.  "
                "fp32 MFMA TFLOP/s = 512 x SQ_INSTS_VALU_MFMA_MOPS_F32 / the average duration of the same launch "
                "shape in the kernel-trace run, against 157.3 TFLOP/s (dense fp32 MFMA peak).\n\n")
        for label, d, trace, detail in zip(args.label, args.dir, args.trace, args.detail):
            fac = agent_facts(d)
            vals = {c: per_kernel(d, c) for c in MFMA_COUNTERS}
            durs = trace_durations(trace) if trace else {}
            sizes = json.load(open(detail))["per_size"] if detail else []
            f.write(f"## {label}\n\n| bench key | kernel | grid | MFMA busy | MFMA instructions | "
                    "fp32 MFMA flop | avg us | fp32 MFMA TFLOP/s | % of 157.3 |\n|---|---|---:|---:|---:|---:|---:|---:|---:|\n")
            for (name, grid) in sorted(vals["GRBM_GUI_ACTIVE"]):
                keys = bench_keys(name, grid, sizes)
                if not keys:
                    continue
                busy = vals["SQ_VALU_MFMA_BUSY_CYCLES"].get((name, grid), 0.0)
                gui = vals["GRBM_GUI_ACTIVE"][(name, grid)] / fac["xcc"]
                util = busy / (gui * fac["simd"]) if gui else 0.0
                flop = 512.0 * vals["SQ_INSTS_VALU_MFMA_MOPS_F32"].get((name, grid), 0.0)
                v = durs.get((name, grid))
                us = sum(v) / len(v) / 1e3 if v else float("nan")
                tf = flop / (us * 1e-6) / 1e12 if v else float("nan")
                for key in keys:
                    f.write(f"| {key.replace('|', chr(92) + '|')} | {name} | {grid} | {util:.1%} | "
                            f"{vals['SQ_INSTS_MFMA'].get((name, grid), 0.0):.0f} | {flop:.3g} | {us:.2f} | "
                            f"{tf:.1f} | {tf / 157.3:.1%} |\n")
            f.write("\n")
    print(f"wrote {args.md}")
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
    c = sub.add_parser("counters")
    c.add_argument("--dir", action="append", required=True, help="output dir of a --pmc run of MFMA_COUNTERS")
    c.add_argument("--trace", action="append", required=True, help="kernel-trace dir of the same command")
    c.add_argument("--detail", action="append", required=True, help="bench_detail.json of the same command")
    c.add_argument("--label", action="append", required=True, help="section title per --dir")
    c.add_argument("--md", required=True)
    c.add_argument("--command", default="")
    args = ap.parse_args()
    if args.cmd == "stats":
        return stats(args)
    if args.cmd == "counters":
        return counters(args)

    fetch = per_kernel(args.fetch, "FETCH_SIZE")
    write = per_kernel(args.write, "WRITE_SIZE")
    f_cal, w_cal = calibration(args.fetch, "FETCH_SIZE"), calibration(args.write, "WRITE_SIZE")
    sq = {c: per_kernel(args.sq, c) for c in SQ_COUNTERS} if args.sq else {}
    durs = trace_durations(args.trace) if args.trace else {}
    sizes = json.load(open(args.detail))["per_size"]

    detail = json.load(open(args.detail))
    real_sizes = detail.get("real_per_size", [])
    rows_out, traffic = [], {}
    for (name, grid) in sorted(set(fetch) | set(write)):
        fb = fetch.get((name, grid), float("nan")) * 1024 / f_cal
        wb = write.get((name, grid), float("nan")) * 1024 / w_cal
        for key in bench_keys(name, grid, sizes):
            traffic[key] = round(fb + wb)
            ept = 16 if name.startswith("mfma_fft_kernel") else 1 << _template_args(name)[1]
            rows_out.append((key, name, grid, 16 * grid * ept, fb, wb))
        for key in real_keys(name, grid, real_sizes):
            # a real-transform launch: bytes it moves per its rows' algorithmic bytes
            rows = int(key.rsplit("=", 1)[1])
            n = int(key.split("|N=")[1].split("|")[0])
            traffic[key] = round(fb + wb)
            rows_out.append((key, name, grid, real_alg_bytes(n) * rows, fb, wb))
    executes = execute_rows(traffic, sizes, real_sizes)

    with open(args.json, "w") as f:
        json.dump(dict(traffic, **{f"execute {e['transform']}|N={e['n']}|B={e['batch']}": e["hbm_bytes"]
                                   for e in executes}), f, indent=1, sort_keys=True)
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
        if executes:
            f.write("\n## Per execute: every launch of one transform call\n\n"
                    "HBM bytes of all launches of one execute (each launch key times its launches per execute) "
                    "over the transform's algorithmic bytes (C2C: 16 N per row; R2C / C2R: 4 N + 8 (N/2 + 1) "
                    "per row).  A ratio of 2 means the data makes two HBM round trips.\n\n")
            f.write("| transform | N | B | flow | launches (kinds) | algorithmic MiB | HBM MiB | HBM / algorithmic |\n")
            f.write("|---|---:|---:|---|---|---:|---:|---:|\n")
            for e in executes:
                f.write(f"| {e['transform']} | {e['n']} | {e['batch']} | {e['flow']} | {', '.join(e['launch_keys'])} | "
                        f"{e['algorithmic_bytes'] / 2**20:.1f} | {e['hbm_bytes'] / 2**20:.1f} | {e['ratio']:.3f} |\n")
    print(f"wrote {args.json} ({len(traffic)} kernels) and {args.md}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
