"""Host logic of kunlunxin-fft_amd/pmc_summary.py on synthetic rocprofv3 CSVs:
copy calibration, (kernel, grid) -> bench-size matching, traffic bytes and
the per-launch-shape duration table."""
import csv
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCRIPT = os.path.join(ROOT, "kunlunxin-fft_amd", "pmc_summary.py")
LDS = "void mfft::(anonymous namespace)::lds_fft_kernel<10, 4, -1, 0>(void const*, void*, float)"
P1 = "void mfft::(anonymous namespace)::fourstep_pass_kernel<10, 5, 4, -1, 0>(float2 const*, int)"
COPY = "__amd_rocclr_copyBuffer"
MIB = 1024  # counter values are KiB


def _counters(path, counter, rows):
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Grid_Size", "Kernel_Name", "Counter_Name", "Counter_Value"])
        for i, (name, grid, kib) in enumerate(rows, 1):
            w.writerow([i, grid, name, counter, kib])


def _detail(path):
    sizes = [{"n": 1024, "batch": 32768, "flow": "lds-fused", "split": None},
             {"n": 1 << 20, "batch": 64, "flow": "four-step", "split": [1024, 1024, 16]}]
    with open(path, "w") as f:
        json.dump({"per_size": sizes}, f)


def test_traffic_calibrates_on_leading_copies(tmp_path):
    # the counters read half (fetch) and all (write) of the bytes moved;
    # a later, larger copy must not change the calibration
    lds_grid, p1_grid = 2097152, 524288  # 2^25 and 2^24 points
    fetch = [(COPY, 131072, 128 * MIB), (COPY, 131072, 128 * MIB), (LDS, lds_grid, 128 * MIB),
             (P1, p1_grid, 64.5 * MIB), (COPY, 131072, 300 * MIB)]
    write = [(COPY, 131072, 256 * MIB), (COPY, 131072, 256 * MIB), (LDS, lds_grid, 256 * MIB),
             (P1, p1_grid, 128 * MIB), (COPY, 131072, 600 * MIB)]
    _counters(tmp_path / "f", "FETCH_SIZE", fetch)
    _counters(tmp_path / "w", "WRITE_SIZE", write)
    _detail(tmp_path / "d.json")
    out = tmp_path / "t.json"
    subprocess.run([sys.executable, SCRIPT, "traffic", "--fetch", str(tmp_path / "f"), "--write",
                    str(tmp_path / "w"), "--detail", str(tmp_path / "d.json"), "--json", str(out),
                    "--md", str(tmp_path / "t.md")], check=True, capture_output=True)
    t = json.load(open(out))
    assert t["lds_fft_kernel|N=1024|rows=32768"] == 512 << 20
    assert t["fourstep_pass_kernel pass 1 (n1=1024)|N=1048576|rows=16"] == (129 + 128) << 20
    assert "scaled by 2.000" in open(tmp_path / "t.md").read()


def test_stats_one_row_per_launch_shape(tmp_path):
    d = tmp_path / "trace"
    d.mkdir()
    rows = [(LDS, 2097152, 100_000), (LDS, 2097152, 102_000), (LDS, 2048, 4_000), (P1, 524288, 64_000)]
    with open(d / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"])
        t = 0
        for name, grid, ns in rows:
            w.writerow([name, t, t + ns, grid, 1, 1])
            t += ns + 1000
    _detail(tmp_path / "d.json")
    md = tmp_path / "s.md"
    subprocess.run([sys.executable, SCRIPT, "stats", "--dir", str(d), "--detail", str(tmp_path / "d.json"),
                    "--md", str(md)], check=True, capture_output=True)
    text = open(md).read()
    assert "| lds_fft_kernel<10, 4, -1, 0> | 2097152 | N=1024\\|rows=32768 | 2 | 0.202 | 101.00 |" in text
    assert "| lds_fft_kernel<10, 4, -1, 0> | 2048 | - | 1 |" in text
    assert "| fourstep_pass_kernel<10, 5, 4, -1, 0> | 524288 | N=1048576\\|rows=16 | 1 |" in text


def test_stats_labels_real_transform_launches(tmp_path):
    """The real-transform leg: LDS R2C/C2R instances, four-step passes over
    the half-length core and the standalone stitch kernel are labelled from
    real_per_size; a plain forward pass of the same shape is not an R2C
    launch."""
    d = tmp_path / "trace"
    d.mkdir()
    r2c = "void mfft::(anonymous namespace)::lds_fft_kernel<9, 4, -1, 1>(void const*, void*, float)"
    p1 = "void mfft::(anonymous namespace)::fourstep_r2c_pass1_kernel<8, 4, 4>(float2 const*, int)"
    plain = "void mfft::(anonymous namespace)::fourstep_pass_kernel<8, 4, 4, -1, 0>(float2 const*, int)"
    st = ("void mfft::(anonymous namespace)::r2c_stitch_kernel(float2 const*, float2*, float2 const*, long, "
          "unsigned int, float)")
    n_lds, b_lds = 1024, 32768           # core 512: 2^24 points, 16 per thread
    n_fs, b_fs = 1 << 16, 512            # core 2^15 = 256 x 128
    pairs = n_fs // 4 + 1                # one stitch thread per mirror pair of the core, flat over the batch
    rows = [(r2c, (n_lds // 2) * b_lds // 16, 50_000), (p1, (n_fs // 2) * b_fs // 16, 60_000),
            (st, (pairs * b_fs + 255) // 256 * 256, 53_000), (plain, (n_fs // 2) * b_fs // 16, 61_000)]
    with open(d / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"])
        t = 0
        for name, grid, ns in rows:
            w.writerow([name, t, t + ns, grid, 1, 1])
            t += ns + 1000
    real = [{"n": n_lds, "batch": b_lds, "transform": "r2c", "flow": "lds-fused", "split": None},
            {"n": n_fs, "batch": b_fs, "transform": "r2c", "flow": "four-step", "split": [256, 128, b_fs]}]
    with open(tmp_path / "d.json", "w") as f:
        json.dump({"per_size": [], "real_per_size": real}, f)
    md = tmp_path / "s.md"
    subprocess.run([sys.executable, SCRIPT, "stats", "--dir", str(d), "--detail", str(tmp_path / "d.json"),
                    "--md", str(md)], check=True, capture_output=True)
    text = open(md).read()
    assert "| r2c N=1024\\|rows=32768 |" in text
    assert "| r2c N=65536\\|rows=512 |" in text
    assert text.count("r2c N=65536") == 2  # pass 1 and the stitch
    assert "| fourstep_pass_kernel<8, 4, 4, -1, 0> | 1048576 | - |" in text


def test_real_keys_label_the_fused_real_passes():
    """R2C pass 1 / pass 2 (stitch) and C2R pass 1 (pre-twiddle) of the
    fused real four-step: labelled by transform and pass from their length
    template argument and the points they cover, never across transforms."""
    from kunlunxin_fft_amd.pmc_summary import real_keys

    n, b = 1 << 16, 512                  # core 2^15 = n1 256 x n2 128
    real = [{"n": n, "batch": b, "transform": t, "flow": "four-step", "split": [256, 128, b]}
            for t in ("r2c", "c2r")]
    pts = (n // 2) * b
    assert real_keys("fourstep_r2c_pass1_kernel<8, 4, 4>", pts >> 4, real) == [f"r2c pass 1|N={n}|rows={b}"]
    assert real_keys("fourstep_r2c_pass2_kernel<7, 3, 4>", pts >> 3, real) == [f"r2c pass 2|N={n}|rows={b}"]
    assert real_keys("fourstep_c2r_pass1_kernel<8, 4, 4>", pts >> 4, real) == [f"c2r pass 1|N={n}|rows={b}"]
    # wrong length for the pass, or a grid that covers other points: no label
    assert real_keys("fourstep_r2c_pass2_kernel<8, 4, 4>", pts >> 4, real) == []
    assert real_keys("fourstep_r2c_pass1_kernel<8, 4, 4>", pts >> 5, real) == []
    # the plain row pass: C2R's inverse pass 2 only; a forward one of the
    # same shape is a C2C launch, not an R2C pass
    assert real_keys("fourstep_pass_kernel<7, 3, 4, 1, 1>", pts >> 3, real) == [f"c2r pass 2|N={n}|rows={b}"]
    assert real_keys("fourstep_pass_kernel<7, 3, 4, -1, 1>", pts >> 3, real) == []
    assert real_keys("fourstep_pass_kernel<8, 4, 4, 1, 0>", pts >> 4, real) == []


def test_execute_rows_sum_every_launch_of_one_execute():
    """Per-execute traffic: each launch key counts batch / rows-per-launch
    times, against 16 N (C2C) or 4 N + 8 (N/2+1) (real) bytes per row."""
    from kunlunxin_fft_amd.pmc_summary import execute_rows, real_alg_bytes

    n, b = 1 << 20, 64
    one = 16 * n * 32  # one 32-row chunk launch moving its rows once
    traffic = {
        f"fourstep_pass_kernel pass 1 (n1=1024)|N={n}|rows=32": one,
        f"fourstep_pass_kernel pass 2 (n2=1024)|N={n}|rows=32": one,
        f"lds_fft_kernel|N=1024|rows=32768": 16 * 1024 * 32768,
        f"r2c pass 1|N={n}|rows=32": 8 * (n // 2) * 2 * 32,
        f"r2c pass 2|N={n}|rows=32": 8 * (n // 2) * 2 * 32,
        f"r2c r2c_stitch_kernel|N={n}|rows=32": real_alg_bytes(n) * 32 // 2 * 3,
    }
    sizes = [{"n": n, "batch": b, "flow": "four-step"}, {"n": 1024, "batch": 32768, "flow": "lds-fused"}]
    real = [{"n": n, "batch": b, "flow": "four-step", "transform": "r2c"}]
    rows = {(e["transform"], e["n"]): e for e in execute_rows(traffic, sizes, real)}
    assert rows[("c2c", n)]["ratio"] == 2.0 and rows[("c2c", n)]["hbm_bytes"] == 4 * one
    assert rows[("c2c", 1024)]["ratio"] == 1.0
    r = rows[("r2c", n)]
    assert r["launch_keys"] == ["r2c pass 1", "r2c pass 2", "r2c r2c_stitch_kernel"]
    assert r["hbm_bytes"] == 2 * (2 * 8 * (n // 2) * 2 * 32 + real_alg_bytes(n) * 32 // 2 * 3)


def test_kernel_names_with_a_boolean_template_argument():
    """The LDS kernel's names carry its staged flag (true / false) as a fifth
    template argument; the size matching reads it as 1 / 0."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("_pmc_summary", SCRIPT)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert mod._template_args("lds_fft_kernel<10, 4, -1, 0, false>") == [10, 4, -1, 0, 0]
    assert mod._template_args("lds_fft_kernel<4, 2, -1, 0, true>") == [4, 2, -1, 0, 1]
    assert mod._template_args("foo<T, 3>") is None
    sizes = [{"n": 1024, "batch": 32768, "flow": "lds-fused", "split": None}]
    assert mod.bench_keys("lds_fft_kernel<10, 4, -1, 0, false>", 2097152, sizes) == \
        ["lds_fft_kernel|N=1024|rows=32768"]
    real = [{"n": 1024, "batch": 32768, "transform": "r2c", "flow": "lds-fused", "split": None}]
    assert mod.real_keys("lds_fft_kernel<9, 4, -1, 1, false>", (512 * 32768) // 16, real) == \
        ["r2c lds_fft_kernel|N=1024|rows=32768"]
