"""bench.py's output contract: the one JSON line the driver parses, and the
refusal of more than one GPU (every box here has one).

The driver reads the line from the tail of stdout, so it must be the last
line and stay a few KB at full size; the per-launch lists, vendor columns
and config-5 cells live in the detail record."""
import importlib.util
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")
KEYS = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
        "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline")


def _bench_module():
    spec = importlib.util.spec_from_file_location("_bench_for_test", BENCH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _full_record(bench):
    """A full-size record as main() assembles it: 11 C2C sizes with launch
    lists and vendor columns, 22 real rows, configs 2-4, all 44 config-5
    cells, roofline, CPU baseline and provenance."""
    per_size, real = [], []
    for n in bench.SIZES:
        b = bench.batch_for(n)
        launches = 4 if n == 1 << 20 else (2 if n >= 1 << 16 else 1)
        per_size.append({"n": n, "batch": b, "executed": "fft_four_step_batch", "flow": "four-step",
                         "fallback": False, "launches": launches, "ms": 0.18104, "gbps": 2965.5,
                         "frac_hbm": 0.3707, "gflops": 14827.7, "launch_ms": [0.09005] * launches,
                         "split": [256, 256, 512], "round_trips": 2, "frac_of_copy_bound": 0.9416,
                         "vendor_ms": 0.38127, "vendor_gbps": 1408.1})
        for tt in ("r2c", "c2r"):
            real.append({"n": n, "batch": b, "transform": tt, "executed": "fft_four_step_batch",
                         "flow": "four-step", "launches": 2, "ms": 0.11378, "gbps": 2359.2, "frac_hbm": 0.2949,
                         "split": [512, 128, 256]})
    lat = {"n": 2048, "batch": 1, "transform": "c2c forward", "executed": "fft_lds_fused",
           "api_wall_p50_ms": 0.04123, "api_wall_mad_ms": 0.00071, "trials": 160, "kernel_event_p50_ms": 0.00612,
           "api_gbps": 0.795, "kernel_gbps": 5.4,
           "graph_replay_us_per_transform": 2.123, "reference_p800_api_p50_ms": 0.4036,
           "api_p50_speedup_vs_reference_p800": 9.8}
    cfg = lambda n, b, t="c2c forward": dict(lat, n=n, batch=b, transform=t)  # noqa: E731
    cells = [{"n": 1 << k, "batch": b, "selected": "fft_lds_fused_batch", "selected_flow": "lds-fused",
              "selection_source": "table", "selected_us": 12.34, "m0": "fft_dit_batch", "m0_us": 45.67,
              "speedup_vs_m0": 3.7, "mfma_candidate": "fft_dit_matrix_batch", "mfma_flow": "dense-mfma",
              "mfma_us": 23.45, "mfma_over_selected": 1.9, "guard_pct": 2.0, "clears_guard": True}
             for k in range(4, 15) for b in (1, 16, 64, 256)]
    return {
        "metric": bench.METRIC, "value": 3838.9, "unit": "GB/s", "n_gpus": 1, "steps": 20, "warmup": 5,
        "ms_per_step": 1.678, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "complex64 (fp32)", "data": "synthetic: iid N(0,1) real/imag parts, fixed device seed",
        "config": {"workload": bench.WORKLOAD, "frac_hbm_of_value": 0.4799, "runner_forced": None,
                   "d2d_copy_gbps": 5012.3, "frac_of_d2d_copy": 0.7659, "stream_copy_gbps": 6301.2,
                   "frac_of_stream_copy": 0.6092},
        "provenance": {"profile_hash": "0123456789abcdef", "env_hash": "fedcba9876543210",
                       "table_sha16": "0" * 16, "table_profile_hash": "0123456789abcdef",
                       "table_env_hash": "fedcba9876543210", "composition_sha16": "1" * 16,
                       "csrc_sha16": "2" * 16, "lib_sha16": "3" * 16, "commit": "abcdef012345",
                       "build_commit": "abcdef012345", "build_dirty": False, "build_matches_csrc": True},
        "roofline": {"bound": "hbm", "achieved": 2810.4, "peak": 8000.0, "unit": "GB/s", "frac": 0.3513,
                     "traffic": 2149580800, "traffic_over_algorithmic": 2.001,
                     "kernel": "fourstep_pass_kernel pass 1 (n1=1024) + fourstep_pass_kernel pass 2 (n2=1024) "
                               "[four-step, N=1048576, B=64, 32 rows per launch, 4 launches per execute, "
                               "counted together]",
                     "algorithmic_bytes_per_execute": 1073741824, "launch_ms": [0.10735, 0.08711, 0.10787, 0.08763],
                     "sum_launch_ms": 0.38996, "share_of_step": 0.232, "copy_ceiling_gbps": 6301.2,
                     "round_trips": 2, "frac_of_copy_bound": 0.8921},
        "cpu_baseline": {"value": 0.1343, "unit": "GB/s", "cores": 1, "cpu_model": "AMD EPYC 9575F 64-Core Processor",
                         "cpu_id": "vendor_id AuthenticAMD cpu family 26 model 2 stepping 1 cpu MHz 3300.000",
                         "host_cpus": 256, "usable_cpus": 16, "kind": "reference",
                         "sample": "16 transforms of each N = 2^10..2^20 (complex<double>, butterfly::fft_dit "
                                   "with its per-stage twiddle rebuild), median of 5 passes, 4.0 s per pass",
                         "gpu_over_cpu": 28584.5,
                         "all_cores": {"value": 1.41, "cores": 16,
                                       "sample": "the same rows split over 16 std::threads (host reports 256 CPUs)"}},
        "latency_n2048_b1": lat,
        "config2": [cfg(n, b) for n in (1024, 2048) for b in (16, 64)],
        "config3": [cfg(n, b, t) for n in (256, 4096) for b in (1, 64)
                    for t in ("c2c inverse", "r2c forward", "c2r inverse")],
        "config4": [cfg(1 << 20, 1), cfg(1 << 16, 256)],
        "config5": cells,
        "per_size": per_size,
        "real_per_size": real,
    }


def test_compact_line_fits_the_driver_tail():
    bench = _bench_module()
    full = _full_record(bench)
    line = bench.compact_line(full, "gpurun_out/bench_detail.json")
    text = json.dumps(line)
    assert len(json.dumps(full)) > 3 * bench.LINE_LIMIT  # the full record would not fit
    assert len(text) < bench.LINE_LIMIT, len(text)
    for k in KEYS:
        assert k in line, k
    assert line["roofline"]["frac"] == 0.3513 and line["roofline"]["traffic_over_algorithmic"] == 2.001
    assert line["cpu_baseline"]["cores"] == 1 and line["cpu_baseline"]["kind"] == "reference"
    assert line["latency_n2048_b1"]["api_wall_p50_ms"] == 0.04123
    assert [r[0] for r in line["per_size"]] == bench.SIZES
    assert all(len(r) == 3 for r in line["per_size"])
    assert [r[0] for r in line["real_per_size"]] == bench.SIZES
    assert all(len(r) == 5 and None not in r for r in line["real_per_size"])
    assert len(line["config3"]) == 12 and len(line["config4"]) == 2
    assert line["config5"]["cells"] == 44 and line["config5"]["clears_guard"] == 44
    assert line["provenance"]["env_hash"] == "fedcba9876543210"
    assert line["provenance"]["build_matches_csrc"] is True and line["config3"] != "in detail record"
    assert line["detail"] == "gpurun_out/bench_detail.json"


def test_compact_line_sheds_rows_before_outgrowing_the_tail():
    bench = _bench_module()
    full = _full_record(bench)
    full["config3"] = full["config3"] * 20  # far more rows than any run makes
    line = bench.compact_line(full)
    assert len(json.dumps(line)) < bench.LINE_LIMIT
    assert line["config3"] == "in detail record" and line["roofline"] is not None


def test_compact_line_of_a_partial_run():
    """Legs switched off leave nulls, never a missing key."""
    bench = _bench_module()
    full = _full_record(bench)
    for k in ("cpu_baseline", "latency_n2048_b1", "config5"):
        full[k] = None
    for k in ("config2", "config3", "config4", "real_per_size"):
        full[k] = []
    line = bench.compact_line(full)
    for k in KEYS:
        assert k in line, k
    assert line["cpu_baseline"] is None and line["config5"] is None and line["real_per_size"] == []


def test_p50_mad_upper_median_convention():
    bench = _bench_module()
    assert bench.p50_mad([1.0, 2.0, 3.0, 10.0]) == (3.0, 2.0)  # p50 = ys[2]; |dev| sorted 0,1,2,7 -> 2
    assert bench.p50_mad([5.0]) == (5.0, 0.0)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_bench_json_line(gpu, tmp_path):
    """Every leg once, as the driver runs it but with 2 steps: the last stdout
    line parses, stays under the driver's tail, and carries the contract keys
    with a measured roofline and CPU baseline; the detail record holds the
    rest."""
    detail = tmp_path / "detail.json"
    r = subprocess.run([sys.executable, BENCH, "--steps", "2", "--warmup", "1", "--detail-out", str(detail)],
                       capture_output=True, text=True, timeout=560, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-2000:]
    last = r.stdout.strip().splitlines()[-1]
    assert len(last) < 4096, len(last)
    line = json.loads(last)
    for k in KEYS:
        assert k in line, k
    assert line["n_gpus"] == 1 and line["steps"] == 2 and line["warmup"] == 1
    assert line["unit"] == "GB/s" and line["higher_is_better"] is True and line["vs_baseline"] is None
    assert 0 < line["value"] < 8000 and line["ms_per_step"] > 0
    assert "workload" in line["config"]
    rf = line["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert 0 < rf["frac"] < 1 and abs(rf["achieved"] / rf["peak"] - rf["frac"]) < 1e-3
    # the measured streaming-copy ceiling, and the dominant flow against it
    assert 3000 < rf["copy_ceiling_gbps"] < 8000 and rf["round_trips"] >= 1
    assert 0 < rf["frac_of_copy_bound"] < 3
    assert line["config"]["stream_copy_gbps"] == rf["copy_ceiling_gbps"]
    cpu = line["cpu_baseline"]
    assert cpu["value"] > 0 and cpu["cores"] == 1 and cpu["kind"] in ("reference", "port")
    assert line["latency_n2048_b1"]["api_wall_p50_ms"] > 0 and line["latency_n2048_b1"]["trials"] == 160
    assert line["latency_n2048_b1"]["api_wall_mad_ms"] >= 0
    assert len(line["per_size"]) == 11 and len(line["real_per_size"]) == 11
    assert line["config5"]["cells"] == 44
    assert line["provenance"]["profile_hash"] and line["provenance"]["csrc_sha16"]
    # the library was built from the sources in this tree
    assert line["provenance"]["build_matches_csrc"] is True and line["provenance"]["build_commit"]
    full = json.loads(detail.read_text())
    assert len(full["config5"]) == 44 and all("launch_ms" in p for p in full["per_size"])
