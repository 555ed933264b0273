"""bench.py's output contract: the one JSON line the driver parses, and the
refusal of more than one GPU (every box here has one)."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


@pytest.mark.gpu
def test_bench_json_line(gpu):
    """A short run over two sizes (one LDS, one four-step): the last stdout
    line carries every key of the contract with sane values."""
    r = subprocess.run([sys.executable, BENCH, "--steps", "2", "--warmup", "1", "--no-cpu", "--no-latency",
                        "--no-vendor", "--no-config5", "--no-real", "--sizes", "1024,65536"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-2000:]
    line = json.loads(r.stdout.strip().splitlines()[-1])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
              "scaling", "vs_baseline", "dtype", "data", "config", "roofline"):
        assert k in line, k
    assert line["n_gpus"] == 1 and line["steps"] == 2 and line["warmup"] == 1
    assert line["unit"] == "GB/s" and line["higher_is_better"] is True and line["vs_baseline"] is None
    assert 0 < line["value"] < 8000 and line["ms_per_step"] > 0
    assert "workload" in line["config"]
    rf = line["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert 0 < rf["frac"] < 1 and abs(rf["achieved"] / rf["peak"] - rf["frac"]) < 1e-3
    # the measured streaming-copy ceiling, and the dominant flow against it
    # (its round trips times the copy time of its bytes; above 1 where the
    # MALL still holds part of the data, as in this two-size cycle)
    assert 3000 < rf["copy_ceiling_gbps"] < 8000 and rf["round_trips"] >= 1
    assert 0 < rf["frac_of_copy_bound"] < 3
    assert line["config"]["stream_copy_gbps"] == rf["copy_ceiling_gbps"]
